"""Pins the oracle (CPU, no GPU): every oracle function is checked against
something independent of its own formula — hand-computed known answers, the
stock transformers modules it restates, brute force on tiny inputs, closed
forms and exact special cases — chosen so that a plausible slip (dropped term,
swapped nibble, wrong axis, wrong order) fails one of them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from oracle import oracle_c
from tests._helpers import Fixed, assert_topk_equivalent, bits_to_bf16_tensor, bf16_bits, norm_err, ulp_diff16


def _bf16_row(x: torch.Tensor) -> np.ndarray:
    return bf16_bits(x.to(torch.bfloat16))


# ------------------------------------------------------------------ RMSNorm
def _stock_rmsnorm(x_bf16: torch.Tensor, w_bf16: torch.Tensor | None, eps: float) -> torch.Tensor:
    """transformers DiffusionGemmaRMSNorm (TF modeling_diffusion_gemma.py:147-165)."""
    from transformers.models.diffusion_gemma.modeling_diffusion_gemma import DiffusionGemmaRMSNorm
    m = DiffusionGemmaRMSNorm(x_bf16.shape[-1], eps=eps, with_scale=w_bf16 is not None)
    if w_bf16 is not None:
        with torch.no_grad():
            m.weight.copy_(w_bf16.float())
    with torch.no_grad():
        return m(x_bf16)


@pytest.mark.parametrize("with_w", [True, False])
def test_rmsnorm_matches_stock_module(with_w):
    g = torch.Generator().manual_seed(5)
    x = (2 * torch.randn(64, 2816, generator=g)).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(2816, generator=g)).to(torch.bfloat16) if with_w else None
    ref = bf16_bits(_stock_rmsnorm(x, w, 1e-6))
    got = mo.rmsnorm(x.float().numpy(), None if w is None else w.float().numpy(), 1e-6)
    d = ulp_diff16(got, ref)
    # torch's fp32 mean and pow(-0.5) may round the last fp32 bit differently
    assert d.max() <= 1
    assert (d == 0).mean() > 0.99


def test_rmsnorm_closed_forms():
    # constant row c: y = c / sqrt(c^2 + eps) * w -> bf16(w) for eps << c^2
    w = torch.tensor([0.5, 2.0, -1.0, 3.0] * 32, dtype=torch.bfloat16)
    x = torch.full((3, 128), 2.0, dtype=torch.bfloat16)
    got = mo.rmsnorm(x.float().numpy(), w.float().numpy(), 1e-6)
    assert np.array_equal(got, np.broadcast_to(bf16_bits(w), got.shape))
    # scale invariance, exact with eps = 0 and a power-of-two factor
    g = torch.Generator().manual_seed(6)
    x = torch.randn(8, 512, generator=g).to(torch.bfloat16)
    a = mo.rmsnorm(x.float().numpy(), None, 0.0)
    b = mo.rmsnorm(4 * x.float().numpy(), None, 0.0)
    assert np.array_equal(a, b)
    # w = None and w = 1 agree; the row rms of the output is ~1
    ones = np.ones(512, dtype=np.float32)
    assert np.array_equal(mo.rmsnorm(x.float().numpy(), ones, 1e-6), mo.rmsnorm(x.float().numpy(), None, 1e-6))
    y = mo.bf16_to_f32(a).astype(np.float64)
    assert np.allclose(np.sqrt((y ** 2).mean(-1)), 1.0, atol=4e-3)
    # eps enters inside the root: an all-zero row stays zero, a tiny row is damped
    z = mo.rmsnorm(np.zeros((1, 128), np.float32), None, 1e-6)
    assert not z.any()
    t = mo.bf16_to_f32(mo.rmsnorm(np.full((1, 128), 1e-3, np.float32), None, 1e-6))
    assert np.allclose(t, 1e-3 / np.sqrt(1e-6 + 1e-6), rtol=1e-2)


# -------------------------------------------------------- W4 pack / dequant
def test_quantize_known_answer():
    # one row, one group of 4: min -1.5, max 3 -> scale 0.3, zero round(1.5/0.3) = 5
    W = np.array([[0.0, 1.5, 3.0, -1.5]], dtype=np.float32)
    q, s, z = mo.quantize_w4(W, 4)
    assert q.tolist() == [[5 | (10 << 4), 15 | (0 << 4)]]  # low nibble = even k
    assert s.dtype == np.float16 and float(s[0, 0]) == 0.300048828125  # fp16(0.3) = 1229/4096
    assert float(z[0, 0]) == 5.0
    Wd = mo.dequant_w4(q, s, z, 4)
    assert Wd.dtype == np.float16
    # 5 * 1229/4096 = 1.50024..., 10 * 1229/4096 = 3.00048...: both round to the fp16 grid point
    assert Wd.tolist() == [[0.0, 1.5, 3.0, -1.5]]
    # a flat group: the scale clamps at 1e-8/15, zero clamps to 0, q to 15, and the
    # fp16 scale underflows, so the group dequantises to 0 (the reference's behaviour)
    q2, s2, z2 = mo.quantize_w4(np.full((1, 4), 2.0, np.float32), 4)
    assert q2.tolist() == [[0xFF, 0xFF]] and float(z2[0, 0]) == 0.0
    assert not mo.dequant_w4(q2, s2, z2, 4).any()


def test_dequant_is_correctly_rounded_product():
    g = np.random.default_rng(7)
    q = g.integers(0, 256, size=(32, 64), dtype=np.uint8)
    s = g.uniform(0.005, 0.02, size=(32, 2)).astype(np.float16)
    z = g.integers(0, 16, size=(32, 2)).astype(np.float16)
    Wd = mo.dequant_w4(q, s, z, 64)
    nib = np.empty((32, 128), np.int64)
    nib[:, 0::2] = q & 15
    nib[:, 1::2] = q >> 4
    exact = (nib - np.repeat(z.astype(np.float64), 64, 1)) * np.repeat(s.astype(np.float64), 64, 1)
    assert np.array_equal(Wd, exact.astype(np.float16))  # one rounding of the exact product
    # unpack is the inverse of the byte packing
    assert np.array_equal(mo.unpack_nibbles(q).astype(np.int64), nib)


def test_quantize_roundtrip_bound():
    g = np.random.default_rng(8)
    W = g.standard_normal((16, 256)).astype(np.float32)
    q, s, z = mo.quantize_w4(W, 128)
    Wd = mo.dequant_w4(q, s, z, 128).astype(np.float32)
    step = np.repeat(s.astype(np.float32), 128, 1)
    assert (np.abs(Wd - W) <= 0.5 * step + 2e-3 * np.abs(W) + 1e-3).all()


# ---------------------------------------------------------------- moe_align
def test_moe_align_known_answer():
    ids = np.array([[1, 0], [0, 2]])
    sr, eids, cap, inv = mo.moe_align(ids, 2, 3)
    assert cap == 10
    assert sr.tolist() == [1, 2, 0, 4, 3, 4, 4, 4, 4, 4]
    assert eids.tolist() == [0, 1, 2, 3, 3]
    assert inv.tolist() == [2, 0, 1, 4]


def _align_brute(ids: np.ndarray, bm: int, E: int):
    flat = np.minimum(ids.reshape(-1), E).tolist()
    n = len(flat)
    max_blocks = (n + bm - 1) // bm + E
    sr = [n] * (max_blocks * bm)
    eids = [E] * max_blocks
    inv = [0] * n
    b = 0
    for e in range(E):
        rows = [r for r in range(n) if flat[r] == e]
        for j, r in enumerate(rows):
            sr[b * bm + j] = r
            inv[r] = b * bm + j
        nb = (len(rows) + bm - 1) // bm
        for k in range(nb):
            eids[b + k] = e
        b += nb
    return np.array(sr), np.array(eids), max_blocks * bm, np.array(inv)


@pytest.mark.parametrize("T,tk,E,bm,seed", [(4, 2, 4, 1, 0), (9, 3, 5, 4, 1), (16, 8, 16, 32, 2), (1, 8, 128, 16, 3),
                                            (33, 2, 3, 8, 4)])
def test_moe_align_brute_force_and_c(T, tk, E, bm, seed):
    g = np.random.default_rng(seed)
    ids = g.integers(0, E, size=(T, tk))
    ids[0, 0] = E          # dropped sentinels, == E and > E
    if T > 1:
        ids[-1, -1] = E + 3
    ref = _align_brute(ids, bm, E)
    got = mo.moe_align(ids, bm, E)
    assert got[2] == ref[2]
    for a, b in zip((got[0], got[1], got[3]), (ref[0], ref[1], ref[3])):
        assert np.array_equal(a, b)
    cg = oracle_c.moe_align(ids, bm, E)
    for a, b in zip((cg[0], cg[1], cg[3]), (ref[0], ref[1], ref[3])):
        assert np.array_equal(a, b)


def test_moe_align_cuda_known_answer():
    """The marlin-capacity align of moe_align_cuda by hand: ids [[1,0],[0,2]],
    block 2, E 3: Nexp 4, mx = 4 + 3*1 = 7, 4 blocks, cap 8; expert 0 holds
    rows 1, 2 (tokens 0, 1), expert 1 row 0 (token 0) and a pad, expert 2 row
    3 (token 1) and a pad."""
    a_row, eids, cap, inv = mo.moe_align_cuda(np.array([[1, 0], [0, 2]]), 2, 3)
    assert cap == 8
    assert a_row.tolist() == [0, 1, 0, 2, 1, 2, 2, 2]
    assert eids.tolist() == [0, 1, 2, 3]
    assert inv.tolist() == [2, 0, 1, 4]
    # fewer rows than experts: mx = min(Nexp * block, Nexp + E * (block - 1))
    a_row, eids, cap, inv = mo.moe_align_cuda(np.array([[5, 1]]), 4, 8)
    assert cap == 8 and eids.tolist() == [1, 5]
    assert a_row.tolist() == [0, 1, 1, 1, 0, 1, 1, 1] and inv.tolist() == [4, 0]


@pytest.mark.parametrize("T,tk,E,bm,seed", [(37, 8, 16, 4, 1), (3, 2, 64, 16, 2), (100, 8, 128, 1, 3),
                                          (512, 8, 128, 64, 4)])
def test_moe_align_cuda_invariants(T, tk, E, bm, seed):
    """Every routed row sits once in its expert's blocks: a_row[inv[r]] is r's
    token, the block of inv[r] carries r's expert, slots past the used blocks are
    padding (T, expert E), and the capacity follows the stated rule."""
    g = np.random.default_rng(seed)
    ids = g.integers(0, E, size=(T, tk))
    a_row, eids, cap, inv = mo.moe_align_cuda(ids, bm, E)
    N = T * tk
    mx = N + E * (bm - 1)
    if N < E:
        mx = min(N * bm, mx)
    assert cap == -(-mx // bm) * bm and eids.size == cap // bm and a_row.size == cap
    flat = ids.reshape(-1)
    assert len(set(inv.tolist())) == N
    assert np.array_equal(a_row[inv], np.arange(N) // tk)
    assert np.array_equal(eids[inv // bm], flat)
    used = int((eids < E).sum()) * bm
    assert used == bm * int(sum(-(-int(c) // bm) for c in np.bincount(flat, minlength=E)))
    assert (a_row[used:] == T).all() and (eids[used // bm:] == E).all()
    pads = np.setdiff1d(np.arange(used), inv)
    assert (a_row[pads] == T).all()


# --------------------------------------------------------------- activations
@pytest.mark.parametrize("act", [mo.ACT_GELU_TANH, mo.ACT_SILU])
def test_activation_closed_forms(act):
    g = np.linspace(-12, 12, 4001).astype(np.float32)
    got = mo.act_fp32(g, act).astype(np.float64)
    ref = mo.act_torch_semantics(g.astype(np.float64), act)
    assert np.allclose(got, ref, rtol=2e-6, atol=2e-6)
    tref = (torch.nn.functional.gelu(torch.from_numpy(g), approximate="tanh") if act == mo.ACT_GELU_TANH
            else torch.nn.functional.silu(torch.from_numpy(g))).numpy()
    assert np.allclose(got, tref, rtol=1e-5, atol=1e-6)
    assert mo.act_fp32(np.float32([0.0]), act)[0] == 0.0


# ---------------------------------------------------------- expert GEMMs
def _experts(E, H, I, seed):
    g = np.random.default_rng(seed)
    gu_q = g.integers(0, 256, size=(E, 2 * I, H // 2), dtype=np.uint8)
    gu_s = g.uniform(0.005, 0.02, size=(E, 2 * I, H // 128)).astype(np.float16)
    gu_z = g.integers(0, 16, size=(E, 2 * I, H // 128)).astype(np.float16)
    dn_q = g.integers(0, 256, size=(E, H, I // 2), dtype=np.uint8)
    dn_s = g.uniform(0.005, 0.02, size=(E, H, I // 64)).astype(np.float16)
    dn_z = g.integers(0, 16, size=(E, H, I // 64)).astype(np.float16)
    return gu_q, gu_s, gu_z, dn_q, dn_s, dn_z


def _dequant_torch(q, s, z, gs):
    """Independent torch form of the W4 dequant: shifts and masks, fp32 product."""
    qt = torch.from_numpy(q.astype(np.int64))
    nib = torch.stack((qt & 15, qt >> 4), dim=-1).reshape(*q.shape[:-1], -1).double()
    zz = torch.from_numpy(z.astype(np.float64)).repeat_interleave(gs, dim=-1)
    ss = torch.from_numpy(s.astype(np.float64)).repeat_interleave(gs, dim=-1)
    return ((nib - zz) * ss).half()


@pytest.mark.parametrize("act", [mo.ACT_GELU_TANH, mo.ACT_SILU])
def test_single_expert_reduces_to_dense_linear(act):
    E, H, I, T = 1, 256, 128, 24
    gu_q, gu_s, gu_z, dn_q, dn_s, dn_z = _experts(E, H, I, 9)
    hidden = torch.randn(T, H, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    ids = np.zeros((T, 1), np.int64)
    w = np.ones((T, 1), np.float32)
    y = mo.moe_forward(hidden.float().numpy(), gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, ids, w, act)
    Wgu = _dequant_torch(gu_q[0], gu_s[0], gu_z[0], 128).double()
    Wdn = _dequant_torch(dn_q[0], dn_s[0], dn_z[0], 64).double()
    A = hidden.half().double()
    gu = torch.nn.functional.linear(A, Wgu).float()
    gate, up = gu[:, :I], gu[:, I:]
    a = torch.nn.functional.gelu(gate, approximate="tanh") if act == mo.ACT_GELU_TANH else torch.nn.functional.silu(gate)
    out2 = (a * up).half()
    out3 = torch.nn.functional.linear(out2.double(), Wdn).float().half()
    mx, mean = norm_err(y, out3.float().numpy())
    assert mx < 2e-3 and mean < 2e-4  # fp32 activation rounding may move an fp16 ulp


def _moe_brute(hidden_f32, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, ids, w, act):
    """Per token, per slot, float64 loops from the packed bytes."""
    T, H = hidden_f32.shape
    E, twoI, _ = gu_q.shape
    I = twoI // 2
    out = np.zeros((T, H), np.float64)
    for t in range(T):
        a = hidden_f32[t].astype(np.float16).astype(np.float64)
        for k in range(ids.shape[1]):
            e = int(ids[t, k])
            Wgu = _dequant_torch(gu_q[e], gu_s[e], gu_z[e], 128).double().numpy()
            Wdn = _dequant_torch(dn_q[e], dn_s[e], dn_z[e], 64).double().numpy()
            g = (Wgu[:I] @ a).astype(np.float32)
            u = (Wgu[I:] @ a).astype(np.float32)
            o2 = (mo.act_torch_semantics(g.astype(np.float64), act) * u).astype(np.float16).astype(np.float64)
            o3 = (Wdn @ o2).astype(np.float32).astype(np.float16).astype(np.float64)
            out[t] += float(np.float32(w[t, k])) * o3
    return out


@pytest.mark.parametrize("act", [mo.ACT_GELU_TANH, mo.ACT_SILU])
def test_moe_forward_brute_force(act):
    E, H, I, T, tk = 4, 128, 64, 6, 2
    ex = _experts(E, H, I, 11)
    g = np.random.default_rng(12)
    hidden = torch.randn(T, H, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16).float().numpy()
    ids = np.stack([g.permutation(E)[:tk] for _ in range(T)]).astype(np.int64)
    w = g.uniform(0.1, 1.0, size=(T, tk)).astype(np.float32)
    y = mo.moe_forward(hidden, *ex, ids, w, act, block_m=4)
    ref = _moe_brute(hidden, *ex, ids, w, act)
    mx, mean = norm_err(y, ref)
    assert mx < 2e-3 and mean < 2e-4
    # the compact per-expert form gives the same bits
    y2, _, _ = mo.moe_forward_per_expert(hidden, *ex, ids, w, act)
    assert np.array_equal(y, y2)


def test_moe_forward_matches_stock_experts_module():
    """transformers DiffusionGemmaTextExperts.forward on the dequantised
    weights, the reference's own kill-test comparator (pack_experts.py:142-156:
    rel_mean < 5e-3, rel_max < 3e-2)."""
    from transformers.models.diffusion_gemma.configuration_diffusion_gemma import DiffusionGemmaTextConfig
    from transformers.models.diffusion_gemma.modeling_diffusion_gemma import DiffusionGemmaTextExperts
    E, H, I, T, tk = 8, 256, 128, 16, 4
    cfg = DiffusionGemmaTextConfig(num_experts=E, hidden_size=H, moe_intermediate_size=I,
                                   hidden_activation="gelu_pytorch_tanh")
    m = DiffusionGemmaTextExperts(cfg)
    ex = _experts(E, H, I, 14)
    gu_q, gu_s, gu_z, dn_q, dn_s, dn_z = ex
    with torch.no_grad():
        m.gate_up_proj.copy_(torch.stack([_dequant_torch(gu_q[e], gu_s[e], gu_z[e], 128) for e in range(E)]).float())
        m.down_proj.copy_(torch.stack([_dequant_torch(dn_q[e], dn_s[e], dn_z[e], 64) for e in range(E)]).float())
    g = torch.Generator().manual_seed(15)
    hidden = torch.randn(T, H, generator=g).to(torch.bfloat16)
    p = torch.softmax(torch.randn(T, E, generator=g), -1)
    w, ids = torch.topk(p, tk, dim=-1)
    w = w / w.sum(-1, keepdim=True)
    with torch.no_grad():
        ref = m(hidden.float(), ids, w).numpy()
    y = mo.moe_forward(hidden.float().numpy(), *ex, ids.numpy(), w.numpy(), mo.ACT_GELU_TANH)
    mx, mean = norm_err(y, ref)
    assert mean < 5e-3 and mx < 3e-2


# ------------------------------------------------------------------ combine
def test_combine_closed_forms_and_c():
    g = np.random.default_rng(16)
    T, tk, H = 5, 4, 64
    out3 = g.standard_normal((T * tk, H)).astype(np.float16)
    inv = g.permutation(T * tk)
    # top-1 with weight 1: the identity gather
    y1 = mo.combine_fma(out3, inv[:T], np.ones((T, 1), np.float32))
    assert np.array_equal(y1, out3[inv[:T]].astype(np.float32))
    # equal weights 1/4 over small-integer rows: the exact mean
    rows = g.integers(-8, 8, size=(T * tk, H)).astype(np.float16)
    ym = mo.combine_fma(rows, inv, np.full((T, tk), 0.25, np.float32))
    ref = rows[inv].astype(np.float64).reshape(T, tk, H).mean(1)
    assert np.array_equal(ym.astype(np.float64), ref)
    # the C fmaf chain and the numpy emulation agree bit for bit; slot order matters
    w = g.uniform(0.0, 1.0, size=(T, tk)).astype(np.float32)
    ybits, yc = oracle_c.combine(out3, inv, w, out_bf16=True)
    yn = mo.combine_fma(out3, inv, w)
    assert np.array_equal(yc, yn)
    assert np.array_equal(ybits, mo.f32_to_bf16(yn))
    yr = mo.combine_fma(out3, inv.reshape(T, tk)[:, ::-1].reshape(-1), w[:, ::-1].copy())
    assert not np.array_equal(yr, yn)  # the other order rounds differently somewhere


def test_bf16_helpers_round_to_nearest_even():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 65504.0, np.nan], np.float32)
    b = mo.f32_to_bf16(x)
    t = bits_to_bf16_tensor(b).float().numpy()
    assert t[0] == 1.0 and t[1] == 1.0 and t[2] == 1.0 + 2 ** -6 and t[3] == -2.5
    assert np.isnan(t[5]) and b[5] == 0x7FC0
    tt = torch.from_numpy(x[:5]).to(torch.bfloat16)
    assert np.array_equal(b[:5], bf16_bits(tt))


# ------------------------------------------------------------------ router
def _stock_router(E, H, k, seed):
    from transformers.models.diffusion_gemma.configuration_diffusion_gemma import DiffusionGemmaTextConfig
    from transformers.models.diffusion_gemma.modeling_diffusion_gemma import DiffusionGemmaTextRouter
    cfg = DiffusionGemmaTextConfig(num_experts=E, hidden_size=H, top_k_experts=k, rms_norm_eps=1e-6)
    m = DiffusionGemmaTextRouter(cfg).to(torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        m.proj.weight.copy_(0.05 * torch.randn(E, H, generator=g))
        m.scale.copy_(1 + 0.1 * torch.randn(H, generator=g))
        m.per_expert_scale.copy_(1 + 0.1 * torch.randn(E, generator=g))
    # the reference patches the router's scale-free norm to the fused RMSNorm
    # (kernels/load_w4_checkpoint.py:126-127); its output is the oracle's rmsnorm
    m.norm.forward = lambda hs: torch.from_numpy(mo.bf16_to_f32(mo.rmsnorm(hs.float().numpy(), None, 1e-6))).to(
        torch.bfloat16)
    return m


def _router_params(m):
    return (m.scale.detach().float().numpy(), m.proj.weight.detach().float().numpy(),
            m.per_expert_scale.detach().float().numpy())


@pytest.mark.parametrize("T,H,E,k,seed", [(64, 512, 32, 4, 31), (48, 2816, 128, 8, 32)])
def test_router_matches_stock_module(T, H, E, k, seed):
    """transformers DiffusionGemmaTextRouter.forward (TF modeling_diffusion_gemma.py:529-548)."""
    m = _stock_router(E, H, k, seed)
    x = (2 * torch.randn(T, H, generator=torch.Generator().manual_seed(seed + 100))).to(torch.bfloat16)
    with torch.no_grad():
        p, w, i = m(x)
    po, wo, io = mo.router(x.float().numpy(), *_router_params(m), 1e-6, k)
    np.testing.assert_allclose(po, p.numpy(), rtol=1e-5, atol=1e-8)
    # equal bf16 scores give exactly equal probabilities; torch.topk orders such
    # ties its own way, the oracle takes the lower id first
    assert_topk_equivalent(po, io, wo, i.numpy(), w.numpy(), rtol=1e-5)
    assert (io == i.numpy()).all(-1).mean() > 0.5


def test_router_closed_forms():
    T, H, E, k = 5, 256, 16, 4
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(33)).to(torch.bfloat16).float().numpy()
    ones_h, ones_e = np.ones(H, np.float32), np.ones(E, np.float32)
    # zero projection: every score 0, probs exactly 1/E; the tie rule takes ids 0..k-1, weights 1/k
    p, w, i = mo.router(x, ones_h, np.zeros((E, H), np.float32), ones_e, 1e-6, k)
    assert np.all(p == np.float32(1.0 / E))
    assert np.array_equal(i, np.broadcast_to(np.arange(k), (T, k)))
    assert np.allclose(w, 1.0 / k)
    # k = E with unit expert scales: the weights are the probabilities, summing to 1
    proj = np.random.default_rng(34).standard_normal((E, H)).astype(np.float32) * 0.05
    p, w, i = mo.router(x, ones_h, proj, ones_e, 1e-6, E)
    assert np.allclose(np.take_along_axis(p, i, -1), w, rtol=1e-6)
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)
    assert np.all(np.diff(w, axis=-1) <= 0)
    # one projection row aligned with a token's normalised row wins for that token,
    # and the per-expert scale multiplies its weight
    proj = np.zeros((E, H), np.float32)
    proj[7] = np.sign(x[2])
    pes = ones_e.copy()
    pes[7] = 2.0
    p, w, i = mo.router(x, ones_h, proj, pes, 1e-6, 1)
    assert i[2, 0] == 7 and w[2, 0] == 2.0


# ------------------------------------------------------------------ block tail
def _oracle_norm_forward(mod):
    # the fused RMSNorm every DiffusionGemmaRMSNorm is patched to
    # (kernels/load_w4_checkpoint.py:126-127); the oracle's rmsnorm restates it
    def fwd(hs):
        w = mod.weight.detach().float().numpy() if mod.with_scale else None
        y = mo.rmsnorm(hs.detach().float().numpy().reshape(-1, hs.shape[-1]), w, mod.eps)
        return bits_to_bf16_tensor(y).reshape(hs.shape)
    return fwd


def stock_layer_tail_case(T, H, seed, ls, ls_dtype, encoder=False):
    """A transformers DiffusionGemma layer (bf16) whose attention, MLP and
    experts return fixed tensors and whose norms are the fused RMSNorm. Returns
    (layer output, m, h1, residual, layer)."""
    from transformers.models.diffusion_gemma.configuration_diffusion_gemma import DiffusionGemmaTextConfig
    from transformers.models.diffusion_gemma import modeling_diffusion_gemma as tfm
    cfg = DiffusionGemmaTextConfig(num_experts=16, hidden_size=H, moe_intermediate_size=128, top_k_experts=4,
                                   intermediate_size=384, num_attention_heads=2, num_key_value_heads=1,
                                   head_dim=128, rms_norm_eps=1e-6, num_hidden_layers=2)
    cls = tfm.DiffusionGemmaEncoderTextLayer if encoder else tfm.DiffusionGemmaDecoderTextLayer
    lay = cls(cfg, 1).to(torch.bfloat16)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for mod in lay.modules():
            if isinstance(mod, tfm.DiffusionGemmaRMSNorm) and mod.with_scale:
                mod.weight.copy_(1 + 0.2 * torch.randn(mod.weight.shape, generator=g))
        lay.layer_scalar = torch.tensor([ls], dtype=ls_dtype)
    for mod in lay.modules():
        if isinstance(mod, tfm.DiffusionGemmaRMSNorm):
            mod.forward = _oracle_norm_forward(mod)
    hidden = torch.randn(1, T, H, generator=g).to(torch.bfloat16)
    m = (10 * torch.randn(T, H, generator=g)).to(torch.bfloat16)
    lay.self_attn = Fixed(torch.randn(1, T, H, generator=g).to(torch.bfloat16), as_tuple=True)
    lay.mlp = Fixed((3 * torch.randn(1, T, H, generator=g)).to(torch.bfloat16))
    lay.experts = Fixed(m)
    seen = {}
    lay.pre_feedforward_layernorm_2.register_forward_pre_hook(lambda mod, a: seen.__setitem__("res", a[0]))
    lay.post_feedforward_layernorm_1.register_forward_hook(lambda mod, a, o: seen.__setitem__("h1", o))
    with torch.no_grad():
        out = lay(hidden)
    return out, m, seen["h1"].reshape(T, H), seen["res"].reshape(T, H), lay


@pytest.mark.parametrize("ls,ls_dtype,encoder", [(0.75, torch.bfloat16, False), (0.7071, torch.float32, False),
                                                 (1.0, torch.bfloat16, True)])
def test_block_tail_matches_stock_layer(ls, ls_dtype, encoder):
    """TF DiffusionGemma{Decoder,Encoder}TextLayer.forward (modeling_diffusion_gemma.py:733-743,
    :655-665) around fixed attention/MLP/expert outputs: bit for bit."""
    T, H = 24, 256
    out, m, h1, res, lay = stock_layer_tail_case(T, H, 41, ls, ls_dtype, encoder)
    lsv = float(lay.layer_scalar.float()[0])
    got = mo.block_tail(bf16_bits(m), h1.float().numpy(), res.float().numpy(),
                        lay.post_feedforward_layernorm_2.weight.float().detach().numpy(),
                        lay.post_feedforward_layernorm.weight.float().detach().numpy(), lsv, 1e-6, 1e-6)
    assert np.array_equal(got, bf16_bits(out.reshape(T, H)))
    # a plausible mix-up fails: the two norm weights swapped
    bad = mo.block_tail(bf16_bits(m), h1.float().numpy(), res.float().numpy(),
                        lay.post_feedforward_layernorm.weight.float().detach().numpy(),
                        lay.post_feedforward_layernorm_2.weight.float().detach().numpy(), lsv, 1e-6, 1e-6)
    assert not np.array_equal(bad, got)


def test_block_tail_closed_forms():
    g = np.random.default_rng(42)
    T, H = 6, 128
    bf = lambda a: mo.f32_to_bf16(np.asarray(a, np.float32))
    m = bf(8 * g.standard_normal((T, H)))
    h1 = mo.bf16_to_f32(bf(g.standard_normal((T, H))))
    res = mo.bf16_to_f32(bf(g.standard_normal((T, H))))
    w2 = mo.bf16_to_f32(bf(1 + 0.2 * g.standard_normal(H)))
    wp = mo.bf16_to_f32(bf(1 + 0.2 * g.standard_normal(H)))
    base = mo.block_tail(m, h1, res, w2, wp, 1.0, 0.0, 1e-6)
    # the first norm is scale-free: with eps 0, 2*m gives the same bits
    m2 = bf(2 * mo.bf16_to_f32(m))
    assert np.array_equal(mo.block_tail(m2, h1, res, w2, wp, 1.0, 0.0, 1e-6), base)
    # the layer scalar: 0 gives zeros, a power of two scales exactly
    assert not mo.bf16_to_f32(mo.block_tail(m, h1, res, w2, wp, 0.0, 0.0, 1e-6)).any()
    y2 = mo.block_tail(m, h1, res, w2, wp, 2.0, 0.0, 1e-6)
    assert np.array_equal(mo.bf16_to_f32(y2), 2 * mo.bf16_to_f32(base))
    # no expert output: the tail is residual + norm(h1)
    z = mo.block_tail(np.zeros((T, H), np.uint16), h1, res, w2, wp, 1.0, 1e-6, 1e-6)
    ref = bf(res + mo.bf16_to_f32(mo.rmsnorm(h1, wp, 1e-6)))
    assert np.array_equal(z, ref)
    # zero residual and hidden_states_1, unit weights: norm(norm(m)) = norm(m) to one ulp
    ones = np.ones(H, np.float32)
    zr = np.zeros((T, H), np.float32)
    nn = mo.block_tail(m, zr, zr, ones, ones, 1.0, 0.0, 0.0)
    assert ulp_diff16(nn, mo.rmsnorm(mo.bf16_to_f32(m), None, 0.0)).max() <= 1



# ------------------------------------------------------------------ tiled down layout
def test_tile_down_known_answer_and_inverse():
    """Hand-checked positions of the tiled layout (I = 192: one 1 KB unit and
    a 512 B tail per 16-row tile) and the inverse round trip for I = 704 / 256."""
    E, H, I = 1, 32, 192
    q = np.arange(E * H * I // 2, dtype=np.int64).reshape(E, H, I // 2)
    t = mo.tile_down(q)
    flat = t.reshape(-1)
    rb = I // 2  # 96 bytes per row
    # tile 0, unit 0, lane c*16 + col = 1*16 + 3 (row 3, bytes 16..31) starts at byte 19*16
    assert flat[19 * 16] == q[0, 3, 16] and flat[19 * 16 + 15] == q[0, 3, 31]
    # tail of tile 0: lane 2*16 + 5 (row 5, bytes 64 + 16 .. +8) at 1024 + 37*8
    assert flat[1024 + 37 * 8] == q[0, 5, 64 + 16] and flat[1024 + 37 * 8 + 7] == q[0, 5, 64 + 23]
    # tile 1 keeps its base address (16 rows later)
    assert flat[16 * rb] == q[0, 16, 0]
    assert sorted(flat.tolist()) == list(range(q.size))  # a permutation
    for I2 in (704, 256):
        qq = np.random.default_rng(I2).integers(0, 256, size=(2, 48, I2 // 2)).astype(np.uint8)
        assert np.array_equal(mo.untile_down(mo.tile_down(qq), I2), qq)


# ------------------------------------------------------------------ MOE_NS down pack
def test_preshuffle_ns_down_brute_force():
    """The NS pack against the reference's stated byte rule
    (kernels/fused_moe_w4_v2.py:183-184: within each 64-K chunk, byte j =
    q[k0+j] | q[k0+32+j] << 4, stored transposed [E, K/2, N]), element by
    element from the unpacked codes; and a hand-checked position."""
    rng = np.random.default_rng(5)
    E, N, K = 2, 8, 192
    codes = rng.integers(0, 16, size=(E, N, K)).astype(np.uint8)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)  # w4a16.py:31
    ns = mo.preshuffle_ns_down(packed)
    assert ns.shape == (E, K // 2, N)
    for e in range(E):
        for n in range(N):
            for kb in range(K // 64):
                for j in range(32):
                    want = codes[e, n, kb * 64 + j] | (codes[e, n, kb * 64 + 32 + j] << 4)
                    assert ns[e, kb * 32 + j, n] == want
    # codes 0..63 of one row: NS byte (kb=0, j=1) holds q[1] = 1 low, q[33] = 33 & 15 = 1 high
    one = (np.arange(64) & 15).astype(np.uint8).reshape(1, 1, 64)
    pk = (one[..., 0::2] | (one[..., 1::2] << 4)).astype(np.uint8)
    assert mo.preshuffle_ns_down(pk)[0, 1, 0] == (1 | (1 << 4))


def test_combine_fma_assumption_at_layer_256():
    """The combine oracle assumes the reference's `acc += w * x` is one FMA per
    slot (Triton contracts it). On a layer_256-shaped combine (256 tokens,
    top-8, H = 2816, softmax top-8 weights) count the outputs that assumption
    decides: about half of the fp32 sums differ from multiply-then-add, and a
    few in 10^5 of the bf16 outputs (28 of 720,896 for this seed), so the
    bit-exact combine claim rests on it for those."""
    g = np.random.default_rng(17)
    T, tk, H = 256, 8, 2816
    out3 = (0.1 * g.standard_normal((T * tk, H))).astype(np.float16)
    inv = g.permutation(T * tk)
    logits = g.standard_normal((T, 128))
    top = np.argsort(-logits, axis=1)[:, :tk]
    p = np.exp(np.take_along_axis(logits, top, 1))
    w = (p / p.sum(1, keepdims=True)).astype(np.float32)
    y_fma = mo.combine_fma(out3, inv, w)
    y_ma = mo.combine_muladd(out3, inv, w)
    frac32 = float((y_fma != y_ma).mean())
    n_bf16 = int((mo.f32_to_bf16(y_fma) != mo.f32_to_bf16(y_ma)).sum())
    n_f16 = int((y_fma.astype(np.float16) != y_ma.astype(np.float16)).sum())
    print(f"FMA vs mul-add: fp32 {frac32:.3f} of outputs differ; bf16 {n_bf16} of {T * H}; fp16 {n_f16}")
    assert 0.3 < frac32 < 0.7
    assert 0 < n_bf16 < T * H // 1000 and n_bf16 < n_f16
    assert np.abs(y_fma - y_ma).max() <= 2 * np.spacing(np.abs(y_fma).max())


# ---------------------------------------------------------------- v1 path
def test_combine_v1_known_answer_and_torch():
    """The v1 combine (kernels/fused_moe_w4.py:125-127). Known answer: w = 0.1
    is fp16 0.0999755859375, times 3 is 0.2999267578125, exactly halfway
    between the fp16 neighbours 1228 and 1229 * 2^-12: round-half-even gives
    0.2998046875 (an fp32 product would keep 0.29992676). Then the reference's
    own expression evaluated by torch on the CPU in fp16 agrees bit for bit
    on random data, and the fp32-chain combine does not (the fp16 roundings
    show)."""
    y = mo.combine_v1(np.array([[3.0]], np.float16), np.array([0]), np.array([[0.1]], np.float32))
    assert y.dtype == np.float16 and float(y[0, 0]) == 0.2998046875
    # two slots: products 0.2998046875 and fp16(0.5 * 2^-11) = 2^-12, fp32 sum, fp16 round
    y2 = mo.combine_v1(np.array([[3.0], [2.0 ** -11]], np.float16), np.array([0, 1]),
                       np.array([[0.1, 0.5]], np.float32))
    assert float(y2[0, 0]) == float(np.float16(0.2998046875 + 2.0 ** -12))
    g = np.random.default_rng(31)
    T, tk, H = 64, 8, 256
    out3 = (0.3 * g.standard_normal((T * tk, H))).astype(np.float16)
    inv = g.permutation(T * tk)
    w = g.dirichlet(np.ones(tk), size=T).astype(np.float32)
    ref = (torch.from_numpy(out3)[torch.from_numpy(inv)].view(T, tk, H)
           * torch.from_numpy(w).to(torch.float16).unsqueeze(-1)).sum(dim=1)
    got = mo.combine_v1(out3, inv, w)
    assert np.array_equal(got.view(np.uint16), ref.numpy().view(np.uint16))
    fma = mo.combine_fma(out3, inv, w).astype(np.float16)
    assert not np.array_equal(got, fma)


def test_moe_forward_v1_matches_v2_for_the_same_activation():
    """With act_fn = tanh-GELU the v1 forward differs from v2 only by where
    the activation is rounded (fp16 gate, fp16 act output, fp16 combine
    products): the two agree to a few fp16 ulps, and v1's out1 is the gate/up
    GEMM the v2 oracle evaluates (gateup_act from the same gate and up)."""
    g = np.random.default_rng(32)
    E, H, I, T, tk = 4, 256, 128, 12, 2
    gu_q, gu_s, gu_z = mo.quantize_w4(g.standard_normal((E * 2 * I, H)).astype(np.float32), mo.GU_GS)
    dn_q, dn_s, dn_z = mo.quantize_w4((0.1 * g.standard_normal((E * H, I))).astype(np.float32), mo.DN_GS)
    gu = [a.reshape(E, 2 * I, -1) for a in (gu_q, gu_s, gu_z)]
    dn = [a.reshape(E, H, -1) for a in (dn_q, dn_s, dn_z)]
    hid = (0.05 * g.standard_normal((T, H))).astype(np.float32)
    ids = np.stack([g.permutation(E)[:tk] for _ in range(T)])
    w = g.dirichlet(np.ones(tk), size=T).astype(np.float32)

    def gelu16(x):
        return torch.nn.functional.gelu(torch.from_numpy(x).float(), approximate="tanh").half().numpy()

    y1 = mo.moe_forward_v1(hid, *gu, *dn, ids, w, gelu16).astype(np.float32)
    y2 = mo.moe_forward_per_expert(hid, *gu, *dn, ids, w, mo.ACT_GELU_TANH)[0]
    assert np.abs(y1 - y2).max() <= 4e-3 * np.abs(y2).max()
    a16 = hid.astype(np.float16)[:3]
    w16 = mo.dequant_w4(gu[0][0], gu[1][0], gu[2][0], mo.GU_GS)
    o1 = mo.gateup_raw(a16, w16)
    assert np.array_equal(o1[:, :I], mo._mm_f32(a16, w16[:I]).astype(np.float16))
    assert np.array_equal(o1[:, I:], mo._mm_f32(a16, w16[I:]).astype(np.float16))


# ---------------------------------------------------------------- packed experts loop
def _stock_loop_torch(out3, inv, ids, w, E, dtype):
    """The reference's packed loop (kernels/pack_experts.py:44-62) evaluated by
    torch on the CPU, with h of (token, slot) = out3[inv[token * tk + slot]]."""
    import torch.nn.functional as F
    T, tk = ids.shape
    o3 = torch.from_numpy(out3)
    inv2 = torch.from_numpy(np.asarray(inv).reshape(T, tk))
    idx = torch.from_numpy(ids)
    tw = torch.from_numpy(w)
    final = torch.zeros(T, out3.shape[1], dtype=dtype)
    expert_mask = F.one_hot(idx, num_classes=E).permute(2, 1, 0)
    hit = torch.greater(expert_mask.sum(dim=(-1, -2)), 0).nonzero()
    for expert_idx in hit:
        e = expert_idx[0]
        top_k_pos, token_idx = torch.where(expert_mask[e])
        h = o3[inv2[token_idx, top_k_pos]]
        h = h * tw[token_idx, top_k_pos, None]
        final.index_add_(0, token_idx, h.to(final.dtype))
    return final


@pytest.mark.parametrize("wdt", [np.float32, np.float16])
@pytest.mark.parametrize("out", ["bf16", "f16", "f32"])
def test_combine_stock_equals_torch_on_the_reference_loop(wdt, out):
    """combine_stock against torch's own CPU evaluation of the reference's
    expression (one_hot mask, per-expert index_add_ of (h * w).to(dtype)), bit
    for bit: experts in ascending id, one rounding per add. A plain slot-order
    fp32 sum rounded once differs (the per-add roundings show)."""
    g = np.random.default_rng(41)
    T, tk, H, E = 48, 8, 128, 16
    out3 = (3.0 * g.standard_normal((T * tk, H))).astype(np.float16)
    inv = g.permutation(T * tk)
    ids = np.stack([g.permutation(E)[:tk] for _ in range(T)]).astype(np.int64)
    w = g.dirichlet(np.ones(tk), size=T).astype(wdt)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[out]
    ref = _stock_loop_torch(out3, inv, ids, w, E, tdt)
    got = mo.combine_stock(out3, inv, ids, w, E, out)
    if out == "bf16":
        assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))
    elif out == "f16":
        assert np.array_equal(got.view(np.uint16), ref.numpy().view(np.uint16))
    else:
        assert np.array_equal(got.view(np.uint32), ref.numpy().view(np.uint32))
    if out == "bf16":
        once = mo.f32_to_bf16(mo.combine_fma(out3, inv, w.astype(np.float32)))
        assert not np.array_equal(got, once)


def test_combine_stock_known_answer():
    """Hand-worked bf16 case: token 0 routed to experts 3 (slot 0, w = 1) and
    1 (slot 1, w = 1) with h = 256 and h = 1.5. Expert 1 goes first: 0 + 1.5
    = 1.5; then 1.5 + 256 = 257.5, which bf16 (8-bit mantissa, ulp 2 at 256)
    rounds to 258 (half to even between 256 + 2 and 256). Slot order would
    give 256 + 1.5 = 257.5 -> 258 as well; with h = 1.0 instead, 1 + 256 =
    257 -> 256 (tie to even) either way, so also: expert 1 term 0.75 and a
    third expert 0 term 0.75 first: 0.75 + 0.75 = 1.5, + 256 -> 258, while
    256 + 0.75 = 256.75 -> 256, + 0.75 -> 256 in slot order."""
    out3 = np.array([[256.0], [0.75], [0.75]], np.float16)
    ids = np.array([[3, 1, 0]], np.int64)
    w = np.ones((1, 3), np.float32)
    got = mo.bf16_to_f32(mo.combine_stock(out3, np.arange(3), ids, w, 4, "bf16"))
    assert float(got[0, 0]) == 258.0
    # skipped ids (>= E) contribute nothing
    got2 = mo.bf16_to_f32(mo.combine_stock(out3, np.arange(3), np.array([[3, 9, 0]], np.int64), w, 4, "bf16"))
    assert float(got2[0, 0]) == 256.0


def test_down_pair_table_known_positions():
    """The tiled layout's (scale, zero) pair table: row r = 16*T + col of
    expert e, group g sits at index ((e*H/16 + T)*G + g)*16 + col, scale bits
    low, zero bits high. Hand-checked entries: expert 1, row 35 (tile 2,
    col 3), group 4 of G = 5, H = 64."""
    E, H, G = 2, 64, 5
    s = (np.arange(E * H * G, dtype=np.float32).reshape(E, H, G) / 1024).astype(np.float16)
    z = (np.arange(E * H * G, dtype=np.float32).reshape(E, H, G) % 16).astype(np.float16)
    t = mo.down_pair_table(s, z)
    assert t.shape == (E * H * G,)
    idx = ((1 * (H // 16) + 2) * G + 4) * 16 + 3
    want = int(s[1, 35, 4].view(np.uint16)) | (int(z[1, 35, 4].view(np.uint16)) << 16)
    assert int(t[idx]) == want
    assert int(t[0]) == int(s[0, 0, 0].view(np.uint16)) | (int(z[0, 0, 0].view(np.uint16)) << 16)
    # a permutation of the pairs: every (row, group) once
    assert len(np.unique(t)) == len(np.unique((s.view(np.uint16).astype(np.uint32) |
                                               (z.view(np.uint16).astype(np.uint32) << 16)).ravel()))
