"""CPU restatement of the fused layer-kernel path (RMSNorm + W4A16 MoE), in numpy.

TEST INFRASTRUCTURE ONLY. This module is the checker: only tests/, the smoke()
entry and the cpu_baseline leg of bench.py may import it. The product path
(the HIP library behind the package) never calls into it.

Every function restates the reference's arithmetic, with the reference
file:line it follows. bf16 values travel as uint16 bit patterns (numpy has no
bf16 type); fp16 values as numpy float16.

Dtype chain restated (kernels/fused_moe_w4_v2.py:96-177, 248-263):
  A      = fp16(hidden)                                  (:347)
  W      = fp16((q - z) * s)  with q, z, s fp16          (:125-128, :172-175)
  g, u   = A @ Wg^T, A @ Wu^T accumulated in fp32         (:128, :135)
  out2   = fp16(act(g) * u), act evaluated in fp32       (:136-138)
  out3   = fp16(out2 @ Wd^T) accumulated in fp32         (:175-177)
  y[t]   = sum_k fp32(w[t,k]) * fp32(out3[inv[t*k+k']])  (:255-263), fixed k order
The fp32 accumulations of the two GEMMs have no defined order in the
reference (Triton tl.dot); this restatement accumulates in float64 and rounds
once to fp32, which is the exact value any fp32 order approximates.
"""
from __future__ import annotations

import numpy as np

GU_GS = 128  # kernels/pack_experts.py:12 (gate/up group size along K=H)
DN_GS = 64   # kernels/pack_experts.py:12 (down group size along K=I)

GELU_C0 = 0.7978845608028654  # sqrt(2/pi), kernels/fused_moe_w4_v2.py:136
GELU_C1 = 0.044715            # kernels/fused_moe_w4_v2.py:136

ACT_GELU_TANH = 0
ACT_SILU = 1


# ----------------------------------------------------------------------------
# bf16 helpers (bit patterns in uint16)
# ----------------------------------------------------------------------------
def f32_to_bf16(x) -> np.ndarray:
    """fp32 -> bf16 bits, round-to-nearest-even; NaN -> 0x7FC0 (torch's rule)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_to_f32(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def f16_to_bf16(x) -> np.ndarray:
    return f32_to_bf16(np.asarray(x, dtype=np.float16).astype(np.float32))


# ----------------------------------------------------------------------------
# RMSNorm — kernels/fused_rmsnorm.py:10-21 (kernel), :24-32 (wrapper)
# ----------------------------------------------------------------------------
def rmsnorm(x32: np.ndarray, w32: np.ndarray | None, eps: float) -> np.ndarray:
    """Returns bf16 bits of shape x32.shape.

    x32: input already converted to fp32 (the kernel's `.to(tl.float32)`, :15).
    ms = sum(x^2)/n + eps in fp32 (:16); the sum is taken exactly (float64)
    and rounded once to fp32. y = x * (1/sqrt(ms)) (:17), then y * w (:19-20),
    each step rounded to fp32, then stored as bf16 (:21).
    """
    x32 = np.asarray(x32, dtype=np.float32)
    n = x32.shape[-1]
    ss = np.sum(x32.astype(np.float64) ** 2, axis=-1, keepdims=True)
    ss32 = ss.astype(np.float32)
    ms = (ss32 / np.float32(n)).astype(np.float32) + np.float32(eps)
    ms = ms.astype(np.float32)
    r = (np.float32(1.0) / np.sqrt(ms.astype(np.float64))).astype(np.float32)
    y = (x32 * r).astype(np.float32)
    if w32 is not None:
        y = (y * np.asarray(w32, dtype=np.float32)).astype(np.float32)
    return f32_to_bf16(y)


# ----------------------------------------------------------------------------
# W4 pack format — kernels/w4a16.py:19-48
# ----------------------------------------------------------------------------
def quantize_w4(W: np.ndarray, gs: int):
    """W[N,K] float -> (q uint8[N,K/2], scale fp16[N,K/gs], zero fp16[N,K/gs]).

    w4a16.py:22-32: per (row, group) scale=(max-min).clamp(1e-8)/15,
    zero=round(-min/scale) clamped to [0,15], q=round(W/scale+zero) clamped;
    byte j = q[2j] | q[2j+1] << 4 (low nibble = even k).
    Rounding is round-half-to-even, as torch.round.
    """
    N, K = W.shape
    assert K % gs == 0
    Wg = W.astype(np.float32).reshape(N, K // gs, gs)
    wmin = Wg.min(-1)
    wmax = Wg.max(-1)
    scale = (np.maximum(wmax - wmin, np.float32(1e-8)) / np.float32(15.0)).astype(np.float32)
    zero = np.clip(np.round(-wmin / scale), 0, 15).astype(np.float32)
    q = np.clip(np.round(Wg / scale[..., None] + zero[..., None]), 0, 15).astype(np.uint8)
    q = q.reshape(N, K)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, scale.astype(np.float16), zero.astype(np.float16)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    """uint8[..., K/2] -> uint8[..., K]; low nibble is the even k (w4a16.py:40-44)."""
    lo = packed & 0xF
    hi = packed >> 4
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def dequant_w4(packed: np.ndarray, scale: np.ndarray, zero: np.ndarray, gs: int) -> np.ndarray:
    """fp16 weights W = fp16((q - z) * s) (w4a16.py:35-48 and the in-kernel
    fp16 form fused_moe_w4_v2.py:125-128). (q - z) is an exact small integer
    and (q - z) * s is exact in fp32, so one rounding to fp16 gives the
    correctly rounded fp16 product, identical to both reference forms."""
    q = unpack_nibbles(packed).astype(np.float32)
    lead = q.shape[:-1]
    K = q.shape[-1]
    q = q.reshape(lead + (K // gs, gs))
    W = (q - zero.astype(np.float32)[..., None]) * scale.astype(np.float32)[..., None]
    return W.reshape(lead + (K,)).astype(np.float16)


def tile_down(dn_q: np.ndarray) -> np.ndarray:
    """The tiled down layout (the load-time repack of this build; the
    reference keeps [E, H, I/2] and repacks only for its own kernel,
    kernels/fused_moe_w4_v2.py:187-206). Per 16-row tile, same base: units
    u < I/128 of 64 lanes x 16 B (lane c*16 + col: row col, bytes
    u*64 + c*16 .. +16), then for I % 128 == 64 a tail of 64 lanes x 8 B
    (row col, bytes (I/128)*64 + c*8 .. +8)."""
    E, H, Ih = dn_q.shape
    g2 = Ih // 64
    t = dn_q.reshape(E, H // 16, 16, Ih)
    main = t[..., :g2 * 64].reshape(E, H // 16, 16, g2, 4, 16).transpose(0, 1, 3, 4, 2, 5).reshape(E, H // 16, -1)
    tail = t[..., g2 * 64:].reshape(E, H // 16, 16, -1, 8).transpose(0, 1, 3, 2, 4).reshape(E, H // 16, -1)
    return np.concatenate([main, tail], axis=-1).reshape(E, H, Ih)


def down_pair_table(dn_s: np.ndarray, dn_z: np.ndarray) -> np.ndarray:
    """The (scale, zero) pair table the tiled layout carries behind its
    weights (this build's load-time repack): per 16-row tile T, group g and
    row col of the tile, uint32 (scale bits | zero bits << 16) at index
    (T * G + g) * 16 + col, G = I / 64."""
    E, H, G = dn_s.shape
    sb = dn_s.astype(np.float16).view(np.uint16).astype(np.uint32)
    zb = dn_z.astype(np.float16).view(np.uint16).astype(np.uint32)
    pairs = (sb | (zb << 16)).reshape(E, H // 16, 16, G)
    return np.ascontiguousarray(pairs.transpose(0, 1, 3, 2)).reshape(-1)


def preshuffle_ns_down(dn_q: np.ndarray, bk: int = 64) -> np.ndarray:
    """The reference's MOE_NS down pack (kernels/fused_moe_w4_v2.py:187-197,
    preshuffle_T_dn): unpack [E, N, K/2] to codes, and within each bk-chunk
    put q[k0 + j] in the low and q[k0 + bk/2 + j] in the high nibble of byte
    j; the result is stored transposed, [E, K/2, N]."""
    E, N, Kh = dn_q.shape
    codes = unpack_nibbles(dn_q).reshape(E, N, (2 * Kh) // bk, bk)
    ns = (codes[..., :bk // 2] | (codes[..., bk // 2:] << 4)).astype(np.uint8).reshape(E, N, Kh)
    return np.ascontiguousarray(ns.transpose(0, 2, 1))


def untile_down(tiled: np.ndarray, I: int) -> np.ndarray:
    """Inverse of tile_down: byte b of tile row r is found at its lane unit."""
    E, H, Ih = tiled.shape
    g2 = I // 128
    out = np.empty_like(tiled)
    flat = tiled.reshape(E, H // 16, 16 * Ih)
    for r in range(16):
        for b in range(Ih):
            if b < g2 * 64:
                u, c, k = b // 64, (b % 64) // 16, b % 16
                src = u * 1024 + (c * 16 + r) * 16 + k
            else:
                bb = b - g2 * 64
                c, k = bb // 8, bb % 8
                src = g2 * 1024 + (c * 16 + r) * 8 + k
            out.reshape(E, H // 16, 16, Ih)[:, :, r, b] = flat[:, :, src]
    return out


def unpack_gateup(pack: np.ndarray, E: int, H: int, I: int):
    """Read the gate/up pack layout of the one-launch expert FFN back into the
    reference buffers (gu_q [E, 2I, H/2] uint8, gu_s / gu_z [E, 2I, H/128]
    fp16). The pack is this build's load-time repack (the reference's
    precedent: kernels/fused_moe_w4_v2.py:187-206). Per expert, unit cb
    (nt = min(11, I/16 - 11 cb) tiles of 16 columns of I), group g: nt*2 blocks
    of 1 KB (block 2w + j, tile w, j = 0 gate / 1 up; lane l = 16 c + col
    holds row j*I + 16 (11 cb + w) + col, bytes 64 g + 16 c .. +16), then
    nt*128 bytes (tile w, column col: s_gate, z_gate, s_up, z_up, fp16)."""
    G = H // 128
    pk = pack.reshape(E, -1)
    q = np.zeros((E, 2 * I, H // 2), np.uint8)
    sc = np.zeros((E, 2 * I, G), np.float16)
    zp = np.zeros((E, 2 * I, G), np.float16)
    off = 0
    for cb in range((I // 16 + 10) // 11):
        nt = min(11, I // 16 - 11 * cb)
        for g in range(G):
            blocks = pk[:, off:off + nt * 2048].reshape(E, nt, 2, 4, 16, 16)   # [e, w, j, c, col, byte]
            sz = pk[:, off + nt * 2048:off + nt * 2176].copy().view(np.float16).reshape(E, nt, 16, 4)
            for w in range(nt):
                for j in range(2):
                    rows = j * I + 16 * (11 * cb + w) + np.arange(16)
                    for c in range(4):
                        q[:, rows, 64 * g + 16 * c:64 * g + 16 * c + 16] = blocks[:, w, j, c]
                    sc[:, rows, g] = sz[:, w, :, 2 * j]
                    zp[:, rows, g] = sz[:, w, :, 2 * j + 1]
            off += nt * 2176
    return q, sc, zp


def unpack_down(pack: np.ndarray, E: int, H: int, I: int):
    """Read the down pack layout back into dn_q [E, H, I/2] uint8 (reference
    layout), dn_s / dn_z [E, H, I/64] fp16. Per expert, unit q (nt = min(22,
    H/16 - 22 q) tiles of 16 columns of H), slot s < I/128: nt blocks of 1 KB
    (tile u; lane l = 16 c + col holds row 16 (22 q + u) + col, bytes
    64 s + 16 c .. +16), then nt*128 bytes (tile u, column col: s, z of group
    2s, then of group 2s + 1); for I % 128 == 64 a tail slot: nt blocks of
    512 B (lane l: bytes 64 (I/128) + 8 c .. +8), then nt*64 bytes (s, z of the
    last group)."""
    Gd, nfull = I // 64, I // 128
    pk = pack.reshape(E, -1)
    q = np.zeros((E, H, I // 2), np.uint8)
    sc = np.zeros((E, H, Gd), np.float16)
    zp = np.zeros((E, H, Gd), np.float16)
    off = 0
    for qb in range((H // 16 + 21) // 22):
        nt = min(22, H // 16 - 22 * qb)
        for sl in range(nfull):
            blocks = pk[:, off:off + nt * 1024].reshape(E, nt, 4, 16, 16)      # [e, u, c, col, byte]
            sz = pk[:, off + nt * 1024:off + nt * 1152].copy().view(np.float16).reshape(E, nt, 16, 2, 2)
            for u in range(nt):
                rows = 16 * (22 * qb + u) + np.arange(16)
                for c in range(4):
                    q[:, rows, 64 * sl + 16 * c:64 * sl + 16 * c + 16] = blocks[:, u, c]
                for h in range(2):
                    sc[:, rows, 2 * sl + h] = sz[:, u, :, h, 0]
                    zp[:, rows, 2 * sl + h] = sz[:, u, :, h, 1]
            off += nt * 1152
        if I % 128:
            blocks = pk[:, off:off + nt * 512].reshape(E, nt, 4, 16, 8)
            sz = pk[:, off + nt * 512:off + nt * 576].copy().view(np.float16).reshape(E, nt, 16, 2)
            for u in range(nt):
                rows = 16 * (22 * qb + u) + np.arange(16)
                for c in range(4):
                    q[:, rows, 64 * nfull + 8 * c:64 * nfull + 8 * c + 8] = blocks[:, u, c]
                sc[:, rows, Gd - 1] = sz[:, u, :, 0]
                zp[:, rows, Gd - 1] = sz[:, u, :, 1]
            off += nt * 576
    return q, sc, zp


# ----------------------------------------------------------------------------
# Routing metadata — kernels/fused_moe_w4.py:15-51 (moe_align)
# ----------------------------------------------------------------------------
def moe_align(topk_ids: np.ndarray, block_m: int, E: int):
    """Returns (sorted_rows int64[cap], expert_ids int64[max_blocks], cap, inv int64[Nexp]).

    fused_moe_w4.py:22 clamps ids to <= E (E = dropped sentinel); :25 stable
    argsort by expert; :28-30 per-expert counts padded to block_m blocks;
    :31-32 fixed capacity; :34 expert_ids = searchsorted(cum, b, right);
    :35-39 sorted position = expert block start + rank within expert;
    :43-50 pad slots hold Nexp, dropped rows map to inv 0.
    """
    topk_ids = np.asarray(topk_ids, dtype=np.int64)
    T, tk = topk_ids.shape
    flat = np.minimum(topk_ids.reshape(-1), E)
    if (flat < 0).any():
        raise IndexError("moe_align: negative expert id")
    Nexp = flat.size
    valid = flat < E
    order = np.argsort(flat, kind="stable")
    sorted_e = flat[order]
    sv = sorted_e < E
    counts = np.bincount(flat[valid], minlength=E)[:E].astype(np.int64)
    nblk = (counts + block_m - 1) // block_m
    max_blocks = (Nexp + block_m - 1) // block_m + E
    cap = max_blocks * block_m
    cum = np.cumsum(nblk)
    expert_ids = np.searchsorted(cum, np.arange(max_blocks), side="right").astype(np.int64)
    dst_start = (cum - nblk) * block_m
    estart = np.cumsum(counts) - counts
    se_c = np.minimum(sorted_e, E - 1)
    pos = np.arange(Nexp) - estart[se_c]
    dst = dst_start[se_c] + pos
    sorted_rows = np.full(cap, Nexp, dtype=np.int64)
    sorted_rows[dst[sv]] = order[sv]
    inv = np.zeros(Nexp, dtype=np.int64)
    inv[order[sv]] = dst[sv]
    return sorted_rows, expert_ids, int(cap), inv


def moe_align_cuda(topk_ids: np.ndarray, block_m: int, E: int):
    """Returns (a_row int32[cap], expert_ids int32[nblk], cap, inv int32[Nexp]).

    The contract of moe_align_cuda (kernels/fused_moe_w4_v2.py:46-76): the same
    expert-ordered, block_m-aligned layout as moe_align, at the capacity
    mx = Nexp + E*(block_m - 1) (min(Nexp*block_m, mx) when Nexp < E, :60-62),
    nblk = ceil(mx / block_m) blocks, cap = nblk * block_m (:63-64); padding
    blocks carry expert id E (:41-43, marlin's -1 folded to E), and
    _align_finalize (:32-43) turns the sorted rows into a_row = row // topk for
    a real row and T for a padding slot, with inv[row] = its sorted position.
    Rows keep their stable order within an expert (the torch align's order).
    """
    topk_ids = np.asarray(topk_ids, dtype=np.int64)
    T, tk = topk_ids.shape
    Nexp = T * tk
    mx = Nexp + E * (block_m - 1)
    if Nexp < E:
        mx = min(Nexp * block_m, mx)
    nblk = (mx + block_m - 1) // block_m
    cap = nblk * block_m
    sr, eids, _, inv = moe_align(topk_ids, block_m, E)
    used_blocks = int((eids < E).sum())
    used = used_blocks * block_m
    a_row = np.full(cap, T, dtype=np.int32)
    s = sr[:used]
    a_row[:used] = np.where(s < Nexp, s // tk, T)
    expert_ids = np.full(nblk, E, dtype=np.int32)
    expert_ids[:used_blocks] = eids[:used_blocks]
    return a_row, expert_ids, int(cap), inv.astype(np.int32)


# ----------------------------------------------------------------------------
# Activations — kernels/fused_moe_w4_v2.py:136-138 (tanh-GELU), SiLU
# ----------------------------------------------------------------------------
def act_fp32(g: np.ndarray, act: int) -> np.ndarray:
    g = g.astype(np.float32)
    if act == ACT_GELU_TANH:
        # 0.5*g*(1+tanh(c0*(g+c1*g^3))) with tanh = 2/(1+exp(-2*inner)) - 1
        inner = np.float32(GELU_C0) * (g + np.float32(GELU_C1) * g * g * g)
        with np.errstate(over="ignore"):
            th = np.float32(2.0) / (np.float32(1.0) + np.exp(np.float32(-2.0) * inner)) - np.float32(1.0)
        return (np.float32(0.5) * g * (np.float32(1.0) + th)).astype(np.float32)
    if act == ACT_SILU:
        with np.errstate(over="ignore"):
            return (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    raise ValueError(f"unknown activation code {act}")


def act_torch_semantics(g64: np.ndarray, act: int) -> np.ndarray:
    """The stock activations (transformers GELUTanh / SiLU) in float64, used as
    the mathematical check on act_fp32."""
    if act == ACT_GELU_TANH:
        return 0.5 * g64 * (1.0 + np.tanh(GELU_C0 * (g64 + GELU_C1 * g64 ** 3)))
    return g64 / (1.0 + np.exp(-g64))


# ----------------------------------------------------------------------------
# Expert GEMMs — kernels/fused_moe_w4_v2.py:96-139 and :146-177
# ----------------------------------------------------------------------------
def _mm_f32(a16: np.ndarray, w16: np.ndarray) -> np.ndarray:
    """fp16 x fp16^T with an exact (float64) accumulate rounded to fp32."""
    return (a16.astype(np.float64) @ w16.astype(np.float64).T).astype(np.float32)


def gateup_act(a16: np.ndarray, gu_w16: np.ndarray, act: int) -> np.ndarray:
    """a16 fp16[M,H]; gu_w16 fp16[2I,H] (gate rows 0..I-1, up rows I..2I-1,
    fused_moe_w4_v2.py:124, :130). Returns out2 fp16[M,I]."""
    I = gu_w16.shape[0] // 2
    g = _mm_f32(a16, gu_w16[:I])
    u = _mm_f32(a16, gu_w16[I:])
    return (act_fp32(g, act) * u).astype(np.float32).astype(np.float16)


def down(out2: np.ndarray, dn_w16: np.ndarray) -> np.ndarray:
    """out2 fp16[M,I]; dn_w16 fp16[H,I]. Returns out3 fp16[M,H] (:175-177)."""
    return _mm_f32(out2, dn_w16).astype(np.float16)


def combine_fma(out3: np.ndarray, inv: np.ndarray, topk_w: np.ndarray) -> np.ndarray:
    """y[t] = fma-chain over k = 0..tk-1 of fp32(w[t,k]) * fp32(out3[inv[t*tk+k]])
    starting from 0 (fused_moe_w4_v2.py:255-259), returned as fp32.
    Each step is one fused multiply-add (Triton contracts `acc += w * x`),
    emulated exactly: w*x is exact in float64 (24+11 bit mantissas) and the
    sum with acc is rounded once to fp32 unless it needs more than 53 bits;
    the C restatement (combine_c in oracle_c.c) uses fmaf and is the bit-exact
    form."""
    T, tk = topk_w.shape
    acc = np.zeros((T, out3.shape[1]), dtype=np.float32)
    w32 = topk_w.astype(np.float32)
    for k in range(tk):
        rows = out3[inv.reshape(T, tk)[:, k]].astype(np.float64)
        acc = (acc.astype(np.float64) + w32[:, k:k + 1].astype(np.float64) * rows).astype(np.float32)
    return acc


def combine_muladd(out3: np.ndarray, inv: np.ndarray, topk_w: np.ndarray) -> np.ndarray:
    """The same chain as combine_fma with `acc += w * x` NOT contracted: the
    product rounded to fp32, then the sum rounded to fp32. Not the reference's
    form; it measures how many outputs the FMA assumption of combine_fma
    decides."""
    T, tk = topk_w.shape
    acc = np.zeros((T, out3.shape[1]), dtype=np.float32)
    w32 = topk_w.astype(np.float32)
    for k in range(tk):
        rows = out3[inv.reshape(T, tk)[:, k]].astype(np.float32)
        acc = (acc + (w32[:, k:k + 1] * rows).astype(np.float32)).astype(np.float32)
    return acc


# ----------------------------------------------------------------------------
# v1 path — kernels/fused_moe_w4.py:54-128 (_grouped_w4 on gate/up, act_fn in
# torch, _grouped_w4 on down, combine in fp16 products)
# ----------------------------------------------------------------------------
def gateup_raw(a16: np.ndarray, gu_w16: np.ndarray) -> np.ndarray:
    """out1 = fp16(A @ W^T) over all 2I gate/up rows (fused_moe_w4.py:87-90
    as :117-118 runs it): fp16 [M, 2I], gate in columns 0..I-1, up in I..2I-1."""
    return _mm_f32(a16, gu_w16).astype(np.float16)


def combine_v1(out3: np.ndarray, inv: np.ndarray, topk_w: np.ndarray) -> np.ndarray:
    """fused_moe_w4.py:125-127: (out3[inv].view(T, tk, H) * w.to(fp16)).sum(1):
    each product fp16(fp16(w) * x) (torch's fp16 multiply: the exact product,
    both factors having 11-bit mantissas, rounded once), the tk products summed
    in fp32 in slot order, the sum rounded to fp16. Returns fp16 [T, H] (the
    caller casts to hidden.dtype, :127)."""
    T, tk = topk_w.shape
    w16 = topk_w.astype(np.float32).astype(np.float16).astype(np.float32)
    acc = np.zeros((T, out3.shape[1]), dtype=np.float32)
    for k in range(tk):
        rows = out3[inv.reshape(T, tk)[:, k]].astype(np.float32)
        acc = acc + (w16[:, k:k + 1] * rows).astype(np.float16).astype(np.float32)
    return acc.astype(np.float16)


def combine_stock(out3: np.ndarray, inv: np.ndarray, topk_ids: np.ndarray, topk_w: np.ndarray, E: int,
                  out_dtype: str = "bf16") -> np.ndarray:
    """The stock experts loop's combine (kernels/pack_experts.py:44-62, TF
    modeling_diffusion_gemma.py:578-588): final = zeros in the hidden dtype;
    for each expert in ascending id, over its (slot, token) pairs,
    final.index_add_(0, token, (h * w[token, slot]).to(dtype)) with h =
    out3[inv[token*tk + slot]] fp16. h * w is fp32 for fp32 / bf16 weights,
    fp16 for fp16 weights (torch's promotion); each add is one rounding to the
    hidden dtype. out_dtype "bf16" returns bf16 bits, "f16" / "f32" arrays."""
    T, tk = topk_ids.shape
    H = out3.shape[1]
    ids = np.asarray(topk_ids, dtype=np.int64)
    inv2 = np.asarray(inv).reshape(T, tk)
    if out_dtype == "bf16":
        rnd = lambda v: bf16_to_f32(f32_to_bf16(v))  # noqa: E731
    elif out_dtype == "f16":
        rnd = lambda v: v.astype(np.float16).astype(np.float32)  # noqa: E731
    else:
        rnd = lambda v: v.astype(np.float32)  # noqa: E731
    acc = np.zeros((T, H), dtype=np.float32)
    for e in range(E):
        ks, ts = np.nonzero((ids == e).T)  # torch.where over the [tk, T] mask: slot-major
        if ts.size == 0:
            continue
        # a token listed twice for one expert is added once per slot, in slot order
        rank = np.zeros(ts.size, dtype=np.int64)
        count: dict = {}
        for i, t in enumerate(ts.tolist()):
            rank[i] = count.get(t, 0)
            count[t] = rank[i] + 1
        for r in range(int(rank.max()) + 1):
            sel = rank == r
            t, k = ts[sel], ks[sel]
            h = out3[inv2[t, k]]
            wk = topk_w[t, k]
            if topk_w.dtype == np.float16:
                term = (h.astype(np.float32) * wk.astype(np.float32)[:, None]).astype(np.float16).astype(np.float32)
            else:
                term = h.astype(np.float32) * wk.astype(np.float32)[:, None]
            acc[t] = rnd(acc[t] + rnd(term))
    if out_dtype == "bf16":
        return f32_to_bf16(acc)
    return acc.astype(np.float16) if out_dtype == "f16" else acc


def _v1_rows(hidden_f32: np.ndarray, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, topk_ids: np.ndarray, act16):
    """out3 rows [T*tk, H] fp16 of the v1 / packed-loop expert stages (row
    t*tk + k for slot k of token t): out1 = fp16(A @ Wgu^T), out2 =
    fp16(act16(gate) * up) (fused_moe_w4.py:117-119; pack_experts.py:56-58),
    out3 = fp16(out2 @ Wd^T)."""
    T, H = hidden_f32.shape
    E, twoI, _ = gu_q.shape
    I = twoI // 2
    tk = topk_ids.shape[1]
    flat = np.asarray(topk_ids, dtype=np.int64).reshape(-1)
    a16 = hidden_f32.astype(np.float16)
    out3_rows = np.zeros((T * tk, H), dtype=np.float16)
    for e in range(E):
        r = np.nonzero(flat == e)[0]
        if r.size == 0:
            continue
        out1 = gateup_raw(a16[r // tk], dequant_w4(gu_q[e], gu_s[e], gu_z[e], GU_GS))
        gate, up = out1[:, :I], out1[:, I:]
        o2 = (np.asarray(act16(gate), dtype=np.float16).astype(np.float32) * up.astype(np.float32)).astype(np.float16)
        out3_rows[r] = down(o2, dequant_w4(dn_q[e], dn_s[e], dn_z[e], DN_GS))
    return out3_rows


def moe_forward_stock(hidden_f32: np.ndarray, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z,
                      topk_ids: np.ndarray, topk_w: np.ndarray, act16, out_dtype: str = "bf16"):
    """One packed_experts_forward call (kernels/pack_experts.py:44-62): the
    v1 expert stages then combine_stock."""
    T, tk = topk_ids.shape
    rows = _v1_rows(hidden_f32, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, topk_ids, act16)
    return combine_stock(rows, np.arange(T * tk), topk_ids, topk_w, gu_q.shape[0], out_dtype)


def moe_forward_v1(hidden_f32: np.ndarray, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z,
                   topk_ids: np.ndarray, topk_w: np.ndarray, act16):
    """One fused_moe_w4 call (fused_moe_w4.py:104-128) with the activation
    act16 (fp16 array -> fp16 array, the module's act_fn): out2 =
    fp16(act16(gate) * up) (:119). Returns the fp16 combine [T, H]. Organised
    per expert; every id must be a real expert."""
    T, H = hidden_f32.shape
    E, twoI, _ = gu_q.shape
    I = twoI // 2
    tk = topk_ids.shape[1]
    flat = np.asarray(topk_ids, dtype=np.int64).reshape(-1)
    a16 = hidden_f32.astype(np.float16)
    out3_rows = np.zeros((T * tk, H), dtype=np.float16)
    for e in range(E):
        r = np.nonzero(flat == e)[0]
        if r.size == 0:
            continue
        out1 = gateup_raw(a16[r // tk], dequant_w4(gu_q[e], gu_s[e], gu_z[e], GU_GS))
        gate, up = out1[:, :I], out1[:, I:]
        o2 = (np.asarray(act16(gate), dtype=np.float16).astype(np.float32) * up.astype(np.float32)).astype(np.float16)
        out3_rows[r] = down(o2, dequant_w4(dn_q[e], dn_s[e], dn_z[e], DN_GS))
    return combine_v1(out3_rows, np.arange(T * tk), topk_w)


def moe_forward(hidden_f32: np.ndarray, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z,
                topk_ids: np.ndarray, topk_w: np.ndarray, act: int,
                block_m: int = 32, return_parts: bool = False):
    """One fused_moe_w4_v2 call (fused_moe_w4_v2.py:319-371), returning fp32
    combine values (the caller rounds to hidden.dtype).

    hidden_f32: the hidden values (bf16 or fp16) already widened to fp32.
    """
    T, H = hidden_f32.shape
    E, twoI, _ = gu_q.shape
    I = twoI // 2
    tk = topk_ids.shape[1]
    assert H % 128 == 0 and I % 64 == 0
    Nexp = T * tk
    sorted_rows, expert_ids, cap, inv = moe_align(topk_ids, block_m, E)
    a16 = hidden_f32.astype(np.float16)                      # :347 hidden.to(fp16)
    out2 = np.zeros((cap, I), dtype=np.float16)
    out3 = np.zeros((cap, H), dtype=np.float16)
    nblk = expert_ids.shape[0]
    for b in range(nblk):
        e = int(expert_ids[b])
        if e >= E:
            continue
        rows = sorted_rows[b * block_m:(b + 1) * block_m]
        valid = rows < Nexp
        if not valid.any():
            continue
        idx = np.nonzero(valid)[0] + b * block_m
        toks = rows[valid] // tk
        gu_w16 = dequant_w4(gu_q[e], gu_s[e], gu_z[e], GU_GS)
        out2[idx] = gateup_act(a16[toks], gu_w16, act)
        dn_w16 = dequant_w4(dn_q[e], dn_s[e], dn_z[e], DN_GS)
        out3[idx] = down(out2[idx], dn_w16)
    y = combine_fma(out3, inv, topk_w)
    if return_parts:
        return y, dict(sorted_rows=sorted_rows, expert_ids=expert_ids, cap=cap, inv=inv,
                       out2=out2, out3=out3)
    return y


def moe_forward_per_expert(hidden_f32, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z,
                           topk_ids, topk_w, act):
    """Same values as moe_forward, organised per expert (compact rows, the
    layout the GPU path uses). Returns (y fp32 [T,H], per-expanded-row out3
    fp16 [T*tk, H]). Rows routed to the dropped sentinel E get zeros."""
    T, H = hidden_f32.shape
    E, twoI, _ = gu_q.shape
    I = twoI // 2
    tk = topk_ids.shape[1]
    flat = np.minimum(np.asarray(topk_ids, dtype=np.int64).reshape(-1), E)
    a16 = hidden_f32.astype(np.float16)
    out3_rows = np.zeros((T * tk, H), dtype=np.float16)
    out2_rows = np.zeros((T * tk, I), dtype=np.float16)
    for e in range(E):
        r = np.nonzero(flat == e)[0]
        if r.size == 0:
            continue
        gu_w16 = dequant_w4(gu_q[e], gu_s[e], gu_z[e], GU_GS)
        dn_w16 = dequant_w4(dn_q[e], dn_s[e], dn_z[e], DN_GS)
        o2 = gateup_act(a16[r // tk], gu_w16, act)
        out2_rows[r] = o2
        out3_rows[r] = down(o2, dn_w16)
    # combine over compact rows: inv = identity on expanded rows
    inv = np.arange(T * tk)
    valid_any = (flat < E)
    if not valid_any.all():
        # reference: dropped rows map to sorted position 0 (the first valid row)
        first = np.nonzero(valid_any)[0]
        if first.size:
            order = np.argsort(flat, kind="stable")
            inv = np.where(valid_any, inv, order[0])
    y = combine_fma(out3_rows, inv, topk_w)
    return y, out2_rows, out3_rows


# ----------------------------------------------------------------------------
# Router — TF modeling_diffusion_gemma.py:529-550 (DiffusionGemmaTextRouter.forward),
# its scale-free norm patched to the fused RMSNorm like every
# DiffusionGemmaRMSNorm (reference kernels/load_w4_checkpoint.py:126-127,
# kernels/fused_rmsnorm.py:35-48).
# ----------------------------------------------------------------------------
def router(x32: np.ndarray, scale32: np.ndarray, proj32: np.ndarray, pes32: np.ndarray, eps: float, k: int):
    """Returns (probs fp32 [T,E], top_k_weights fp32 [T,k], top_k_index int64 [T,k]).

    x32: hidden rows as fp32 (bf16 values); scale32 [H], proj32 [E,H],
    pes32 [E]: the bf16 parameters as fp32.
      y      = bf16(rmsnorm(x))                      norm, with_scale=False (:530)
      h1     = bf16(y * scale)                       bf16 * bf16 (:531)
      h      = bf16(h1 * fp32(H ** -0.5))            bf16 * python scalar (:531)
      scores = bf16(h @ proj^T), fp32 accumulate     nn.Linear in bf16 (:533)
      probs  = softmax(fp32(scores))                 (:535)
      w, idx = top-k of probs, descending            (:538-542); equal values: lower index first
      w      = w / sum(w) * fp32(per_expert_scale[idx])   (:545, :548)
    The GEMM accumulates in float64, rounded once to fp32 (any fp32 order
    approximates that value); softmax likewise in float64, rounded to fp32.
    """
    x32 = np.asarray(x32, dtype=np.float32)
    H = x32.shape[-1]
    y = bf16_to_f32(rmsnorm(x32, None, eps))
    h1 = bf16_to_f32(f32_to_bf16((y * np.asarray(scale32, dtype=np.float32)).astype(np.float32)))
    h = bf16_to_f32(f32_to_bf16((h1 * np.float32(H ** -0.5)).astype(np.float32)))
    sc = (h.astype(np.float64) @ np.asarray(proj32, dtype=np.float64).T).astype(np.float32)
    s = bf16_to_f32(f32_to_bf16(sc)).astype(np.float64)
    e = np.exp(s - s.max(axis=-1, keepdims=True))
    probs = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    idx = np.argsort(-probs, axis=-1, kind="stable")[:, :k].astype(np.int64)
    w = np.take_along_axis(probs, idx, axis=-1)
    w = (w / w.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    w = (w * np.asarray(pes32, dtype=np.float32)[idx]).astype(np.float32)
    return probs, w, idx


# ----------------------------------------------------------------------------
# Feed-forward block tail, the step after the MoE — TF
# modeling_diffusion_gemma.py:733-743 (DiffusionGemmaDecoderTextLayer.forward;
# DiffusionGemmaEncoderTextLayer.forward :655-665 is the same), its RMSNorms
# patched to the fused RMSNorm (kernels/load_w4_checkpoint.py:126-127).
# ----------------------------------------------------------------------------
def block_tail(m_bits: np.ndarray, h1_32: np.ndarray, res32: np.ndarray, post2_w32: np.ndarray,
               post_w32: np.ndarray, ls: float, eps2: float, eps: float) -> np.ndarray:
    """Returns the layer output as bf16 bits [T, H].

    m_bits: the experts' output as bf16 bits (fused_moe_w4_v2 returns the
    hidden dtype, kernels/fused_moe_w4_v2.py:260-263); h1_32, res32: the bf16
    hidden_states_1 and residual as fp32; post2_w32, post_w32: the bf16 norm
    weights as fp32; ls: the layer scalar's value.
      n2 = rmsnorm(m, post2_w)       post_feedforward_layernorm_2 (:735)
      s  = bf16(h1 + n2)             bf16 + bf16, fp32 sum (:738)
      n  = rmsnorm(s, post_w)        post_feedforward_layernorm (:740)
      o  = bf16(res + n)             (:741)
      y  = bf16(o * ls)              hidden_states *= layer_scalar, fp32 product (:743)
    """
    m32 = bf16_to_f32(m_bits)
    n2 = bf16_to_f32(rmsnorm(m32, post2_w32, eps2))
    s = bf16_to_f32(f32_to_bf16((np.asarray(h1_32, dtype=np.float32) + n2).astype(np.float32)))
    n = bf16_to_f32(rmsnorm(s, post_w32, eps))
    o = bf16_to_f32(f32_to_bf16((np.asarray(res32, dtype=np.float32) + n).astype(np.float32)))
    return f32_to_bf16((o * np.float32(ls)).astype(np.float32))


# ----------------------------------------------------------------------------
# Synthetic inputs (the workload definitions) — torch CPU generators so CPU and
# GPU see identical bits.
# ----------------------------------------------------------------------------
def route_softmax_topk(logits: np.ndarray, k: int):
    """softmax(fp32) -> top-k -> renormalise (TF modeling_diffusion_gemma.py:538-547,
    per_expert_scale = 1). Uses torch.topk on CPU for its tie order."""
    import torch
    lg = torch.from_numpy(np.ascontiguousarray(logits, dtype=np.float32))
    p = torch.softmax(lg, dim=-1, dtype=torch.float32)
    w, idx = torch.topk(p, k=k, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return idx.numpy().astype(np.int64), w.numpy().astype(np.float32)
