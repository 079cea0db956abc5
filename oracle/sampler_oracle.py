"""CPU restatement of the per-step sampler pass (entropy + Gumbel-max sample +
argmax over [rows, V] logits), in numpy.

TEST INFRASTRUCTURE ONLY. This module is the checker: only tests/, the smoke()
entry and bench.py's cpu_baseline leg may import it. The product path (the HIP
library behind the package) never calls into it.

Reference: kernels/fused_sampler_ops.py:22-51 (entropy), :54-93 (Gumbel-max
sample and argmax). The noise is Triton's `tl.rand(seed + row, col)`; Triton
is a dependency of the reference (not shipped in it; triton 3.6.0 here), and
its generator is restated from its published algorithm, Philox4x32-10
(Salmon et al., "Parallel random numbers: as easy as 1, 2, 3", SC 2011) with
Triton's counter/key convention and uint -> float conversion
(triton/language/random.py: philox_impl, philox, randint4x, rand,
uint_to_uniform_float).
"""
from __future__ import annotations

import numpy as np

PHILOX_ROUND_A = np.uint64(0xD2511F53)
PHILOX_ROUND_B = np.uint64(0xCD9E8D57)
PHILOX_KEY_A = 0x9E3779B9
PHILOX_KEY_B = 0xBB67AE85
U32 = np.uint64(0xFFFFFFFF)

UNIFORM_SCALE = np.float32(4.6566127342e-10)  # triton uint_to_uniform_float, 32-bit branch
U_LO = np.float32(1e-10)                      # fused_sampler_ops.py:68 clamp
U_HI = np.float32(1.0 - 1e-7)


def philox4x32(c0, c1, c2, c3, k0: int, k1: int, rounds: int = 10):
    """Philox4x32 with `rounds` rounds on uint32 counters (arrays) and a key.
    Each round: (hi, lo) = 0xD2511F53 * c0, (hi', lo') = 0xCD9E8D57 * c2;
    c = (hi' ^ c1 ^ k0, lo', hi ^ c3 ^ k1, lo); then the key is raised by
    (0x9E3779B9, 0xBB67AE85) (triton philox_impl)."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint64) & U32 for c in (c0, c1, c2, c3))
    k0 = np.uint64(k0 & 0xFFFFFFFF)
    k1 = np.uint64(k1 & 0xFFFFFFFF)
    for _ in range(rounds):
        p0 = PHILOX_ROUND_A * c0
        p2 = PHILOX_ROUND_B * c2
        n0 = ((p2 >> np.uint64(32)) ^ c1 ^ k0) & U32
        n2 = ((p0 >> np.uint64(32)) ^ c3 ^ k1) & U32
        c1 = p2 & U32
        c3 = p0 & U32
        c0, c2 = n0, n2
        k0 = (k0 + np.uint64(PHILOX_KEY_A)) & U32
        k1 = (k1 + np.uint64(PHILOX_KEY_B)) & U32
    return (c0.astype(np.uint32), c1.astype(np.uint32), c2.astype(np.uint32), c3.astype(np.uint32))


def row_key(seed: int, row: int):
    """Key of row `row` for the kernel argument `seed` (fused_sampler_ops.py:67,
    `seed + row`). Triton passes an integer argument that fits int32 as int32,
    so seed + row wraps in int32 and is sign-extended to uint64; a wider seed
    is int64. Returns (k0, k1) = (low, high) 32 bits (triton philox)."""
    if -2 ** 31 <= seed < 2 ** 31:
        s = (seed + row) & 0xFFFFFFFF
        if s >= 2 ** 31:
            s -= 2 ** 32
    else:
        s = seed + row
    u = s & 0xFFFFFFFFFFFFFFFF
    return u & 0xFFFFFFFF, u >> 32


def uint_to_uniform_float(x) -> np.ndarray:
    """Triton's conversion of a uint32 to [0, 1): bitcast to int32, negative
    values mapped to -x - 1, times 4.6566127342e-10 in fp32."""
    i = np.asarray(x, dtype=np.uint32).view(np.int32).astype(np.int64)
    i = np.where(i < 0, -i - 1, i)
    return (i.astype(np.float32) * UNIFORM_SCALE).astype(np.float32)


def tl_rand(seed: int, row: int, cols, fast: bool = False) -> np.ndarray:
    """tl.rand(seed + row, cols) for int32 column offsets: Philox4x32-10 on the
    counter (col, 0, 0, 0) with the row key; the first output word to [0, 1).
    fast: the same words from the C restatement (oracle_c.philox_first)."""
    k0, k1 = row_key(seed, row)
    c = np.asarray(cols, dtype=np.int64) & 0xFFFFFFFF
    if fast:
        from oracle import oracle_c
        r0 = oracle_c.philox_first(c.astype(np.uint32), k0, k1)
    else:
        z = np.zeros_like(c)
        r0, _, _, _ = philox4x32(c, z, z, z, k0, k1)
    return uint_to_uniform_float(r0)


def gumbel_noise(u) -> np.ndarray:
    """g = -log(-log(clamp(u, 1e-10, 1 - 1e-7))) in fp32 (fused_sampler_ops.py:68-69)."""
    u = np.minimum(np.maximum(np.asarray(u, dtype=np.float32), U_LO), U_HI)
    return (-np.log(-np.log(u))).astype(np.float32)


def gumbel_argmax(x: np.ndarray, seed: int, fast: bool = False):
    """(sampled index, argmax index) per row (fused_sampler_ops.py:54-93):
    sample = first index of the max of fp32(x + g), g the row's Gumbel noise;
    argmax = first index of the max of x. Returns int64 arrays and the noisy
    scores' top-two margin per row (the gap a different fp32 log could close).
    fast: Philox words from the C restatement."""
    x = np.asarray(x, dtype=np.float32)
    rows, V = x.shape
    samp = np.zeros(rows, dtype=np.int64)
    amax = np.zeros(rows, dtype=np.int64)
    margin = np.zeros(rows, dtype=np.float64)
    cols = np.arange(V, dtype=np.int64)
    for r in range(rows):
        g = gumbel_noise(tl_rand(seed, r, cols, fast=fast))
        xg = (x[r] + g).astype(np.float32)
        samp[r] = int(np.argmax(xg))
        amax[r] = int(np.argmax(x[r]))
        top2 = np.partition(xg.astype(np.float64), V - 2)[V - 2:] if V >= 2 else np.array([0.0, np.inf])
        margin[r] = float(top2[1] - top2[0])
    return samp, amax, margin


def entropy(x: np.ndarray) -> np.ndarray:
    """Entropy in nats of softmax(x) per row, exact (float64), returned as fp32:
    H = logsumexp(x) - sum(p * x) (fused_sampler_ops.py:22-40). Entries equal
    to -inf contribute nothing (p = 0), as in torch's Categorical.entropy."""
    x = np.asarray(x, dtype=np.float64)
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    s = e.sum(axis=-1, keepdims=True)
    lse = m + np.log(s)
    xe = np.zeros_like(x)
    np.multiply(x, e, out=xe, where=e > 0)
    h = lse[..., 0] - xe.sum(axis=-1) / s[..., 0]
    return h.astype(np.float32)
