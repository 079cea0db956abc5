"""CPU checks of the sampler oracle (oracle/sampler_oracle.py), the sampler's
host glue (fast_sampler) and its C ABI argument checks (no GPU).

Pinning of the oracle: Philox4x32-10 against the published Random123
known-answer vectors and against Triton's own tl.rand / tl.randint outputs
(tests/golden/sampler_rand.npz); the uint -> float conversion and the row key
by closed forms; entropy against torch's Categorical.entropy; the Gumbel-max
draw by its distribution (the reference's kill-test band,
kernels/fused_sampler_ops.py:112-122) and its argmax by numpy.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import oracle_c
from oracle import sampler_oracle as so
from tests.conftest import ROOT, load_mod

GOLDEN = os.path.join(ROOT, "tests", "golden", "sampler_rand.npz")

# Random123 kat_vectors, philox4x32 with 10 rounds: counter, key -> output
PHILOX_KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,out", PHILOX_KAT)
def test_philox_known_answers(ctr, key, out):
    got = so.philox4x32(*[np.array([c], dtype=np.uint64) for c in ctr], key[0], key[1])
    assert tuple(int(g[0]) for g in got) == out
    if ctr[1:] == (0, 0, 0):
        assert int(oracle_c.philox_first(np.array([ctr[0]], np.uint32), *key)[0]) == out[0]


def test_philox_c_and_numpy_agree():
    c = np.random.default_rng(3).integers(0, 2 ** 32, size=5000, dtype=np.uint64)
    for k0, k1 in ((0, 0), (123456789, 0xFFFFFFFF), (0xDEADBEEF, 7)):
        z = np.zeros_like(c)
        a = so.philox4x32(c, z, z, z, k0, k1)[0]
        b = oracle_c.philox_first(c.astype(np.uint32), k0, k1)
        assert np.array_equal(a, b)


def test_tl_rand_matches_triton_fixture():
    """Every fixture value of Triton's tl.rand / tl.randint(seed + row, col),
    including seed + row wrapping in int32 (2^31 - 3 + 3) and an int64 seed."""
    d = np.load(GOLDEN)
    cols = d["cols"]
    n = 0
    for si, seed in enumerate(d["seeds"]):
        for r in range(d["rand"].shape[1]):
            k0, k1 = so.row_key(int(seed), r)
            c = cols.astype(np.int64) & 0xFFFFFFFF
            z = np.zeros_like(c)
            assert np.array_equal(so.philox4x32(c, z, z, z, k0, k1)[0], d["randint"][si, r])
            u = so.tl_rand(int(seed), r, cols)
            assert np.array_equal(u.view(np.uint32), d["rand"][si, r].view(np.uint32))
            n += cols.size
    assert n >= 2000


def test_uniform_conversion_and_row_key_closed_forms():
    x = np.array([0, 1, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF], dtype=np.uint32)
    u = so.uint_to_uniform_float(x)
    top = np.float32(2 ** 31 - 1) * so.UNIFORM_SCALE
    assert u[0] == 0.0 and u[4] == 0.0           # int32 -1 -> 0
    assert u[2] == top and u[3] == top and top < 1.0  # INT_MIN -> INT_MAX
    assert u[1] == so.UNIFORM_SCALE
    assert so.row_key(5, 2) == (7, 0)
    assert so.row_key(2 ** 31 - 3, 3) == (0x80000000, 0xFFFFFFFF)  # int32 wrap, sign-extended
    assert so.row_key(-1, 0) == (0xFFFFFFFF, 0xFFFFFFFF)
    assert so.row_key(2 ** 40 + 5, 1) == (6, 256)                  # int64 seed


def test_entropy_matches_torch_categorical():
    g = torch.Generator().manual_seed(11)
    x = (3 * torch.randn(5, 4097, generator=g)).double()
    x[1, ::7] = -float("inf")                                      # masked tokens: p = 0
    ref = torch.distributions.Categorical(logits=x).entropy().numpy()
    got = so.entropy(x.numpy())
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    # uniform logits: log V exactly; one dominant logit: ~0
    assert abs(float(so.entropy(np.zeros((1, 1000)))[0]) - np.log(1000)) < 1e-6
    assert float(so.entropy(np.array([[0.0, -200.0, -200.0]]))[0]) < 1e-80 + 1e-30


def test_gumbel_argmax_distribution_and_argmax():
    """The reference's kill test (kernels/fused_sampler_ops.py:112-122): 4000
    draws of a 1000-token row peaked on 4 tokens stay within a 3-sigma band of
    softmax; the argmax is numpy's (first index of the max)."""
    xp = np.full((1, 1000), -8.0, dtype=np.float32)
    xp[0, :4] = [3.0, 2.0, 1.0, 0.0]
    p_true = np.exp(xp[0].astype(np.float64) - xp[0].max())
    p_true = (p_true / p_true.sum())[:4]
    n = 4000
    counts = np.zeros(1000)
    for i in range(n):
        s, a, _ = so.gumbel_argmax(xp, i * 7919, fast=True)
        counts[s[0]] += 1
        assert a[0] == 0
    p = counts[:4] / n
    tol = 3 * np.sqrt(p_true * (1 - p_true) / n) + 1e-3
    assert (np.abs(p - p_true) <= tol).all(), (p, p_true)
    # the same seed gives the same draw, another seed a different stream
    x = np.random.default_rng(5).standard_normal((3, 5000)).astype(np.float32)
    s1, a1, _ = so.gumbel_argmax(x, 42, fast=True)
    s2, _, _ = so.gumbel_argmax(x, 42)
    assert np.array_equal(s1, s2) and np.array_equal(a1, x.argmax(-1))
    s3, _, _ = so.gumbel_argmax(x, 43, fast=True)
    assert not np.array_equal(s1, s3)


# ------------------------------------------------------------------ host glue
def _sampler(entropy_bound=1.0):
    from transformers.models.diffusion_gemma import generation_diffusion_gemma as G
    smp = G.EntropyBoundSampler.__new__(G.EntropyBoundSampler)
    smp.entropy_bound = entropy_bound
    return G, smp


def test_fast_sampler_bitwise_tier_is_stock():
    """install(parity=False) caches the sampler's entropy for the stopping
    criterion; accept_canvas and the criterion give the stock results bit for bit."""
    fs = load_mod("fast_sampler")
    G, smp = _sampler(1.5)
    stock_accept = G.EntropyBoundSampler.accept_canvas
    stock_call = G.StableAndConfidentStoppingCriteria.__call__
    g = torch.Generator().manual_seed(12)
    logits = 2 * torch.randn(2, 16, 50, generator=g)
    cur = torch.randint(0, 50, (2, 16), generator=g)
    den = torch.randint(0, 50, (2, 16), generator=g)
    ref = G.EntropyBoundSampler.accept_canvas(smp, cur, den, logits, 3)
    crit = G.StableAndConfidentStoppingCriteria.__new__(G.StableAndConfidentStoppingCriteria)
    crit.stability_threshold, crit.confidence_threshold, crit.argmax_canvas_history = 0, 3.0, None
    ref_stop = G.StableAndConfidentStoppingCriteria.__call__(crit, logits.argmax(-1), logits)
    fs.install(parity=False)
    try:
        with pytest.raises(RuntimeError):
            fs.install(parity=True)
        out = G.EntropyBoundSampler.accept_canvas(smp, cur, den, logits, 3)
        stop = G.StableAndConfidentStoppingCriteria.__call__(crit, logits.argmax(-1), logits)
        assert torch.equal(out, ref) and torch.equal(stop, ref_stop)
        assert fs.stats()["hits"] == 1
        logits.add_(0.0)  # a new version of the tensor: the cache misses
        G.StableAndConfidentStoppingCriteria.__call__(crit, logits.argmax(-1), logits)
        assert fs.stats()["misses"] == 1
        assert fs.installed() is False
    finally:
        fs.uninstall()
    assert fs.installed() is None
    assert G.EntropyBoundSampler.accept_canvas is stock_accept
    assert G.StableAndConfidentStoppingCriteria.__call__ is stock_call
    assert fs.stats() == {"hits": 1, "misses": 1}


def test_sampler_abi_rejects_bad_arguments_without_launching():
    L = load_mod("_lib").load()
    P = ctypes.c_void_p
    fake, null = P(1 << 20), P(0)
    assert L.ksl_entropy(null, 0, 0, 100, 100, null, null) == 0          # no rows: no-op
    assert L.ksl_entropy(null, 0, 4, 100, 100, fake, null) == 1          # null logits
    assert L.ksl_entropy(fake, 0, 4, 100, 99, fake, null) == 2           # stride < V
    assert L.ksl_entropy(fake, 0, 4, 2 ** 31, 2 ** 31, fake, null) == 2  # V >= 2^31
    assert L.ksl_entropy(fake, 9, 4, 100, 100, fake, null) == 1          # dtype
    assert L.ksl_gumbel_argmax(fake, 0, 4, 100, 100, 1, fake, null, null) == 1  # argmax output required
    assert L.ksl_sample_step(fake, 0, 4, 0, 100, 1, fake, fake, fake, null) == 2  # V = 0
