"""GPU checks of the reference interface names around the hot path that the
drop-in modules export besides the forwards themselves, through the C ABI:

- w4a16.dequant_w4 (kernels/w4a16.py:35-48): bit-exact vs the oracle;
- fused_moe_w4_v2.preshuffle_T_dn / enable_ns_down (kernels/fused_moe_w4_v2.py:
  186-206): the NS bytes equal the oracle's byte for byte, and a module
  switched by enable_ns_down (or arriving as an NS pack) gives the plain
  pack's output bits;
- pack_experts.fused_experts_forward's MOE_V2 dispatch and MOE_STATS probe
  (kernels/pack_experts.py:14-31, 65-84);
- pack_experts.pack_experts_module(exp, free_bf16, fused) and
  packed_experts_forward (kernels/pack_experts.py:44-62, 87-106), whose
  combine (ksl_moe_combine_stock) is bit-exact vs the oracle given out3;
- the load-time repack caches bind a module only to its own weights, also
  when a freed buffer's address is reused.
"""
import io
import contextlib

import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from tests._helpers import check_norm_err
from tests.conftest import load_mod, load_pkg

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _experts_np(exp):
    return [_np(getattr(exp, k)) for k in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z")]


def _relu_sq(x):
    return torch.relu(x) ** 2


@pytest.mark.parametrize("shape,gs,frac_zero", [((2, 64, 2816), 128, False), ((48, 704), 64, False),
                                                ((1, 16, 256), 32, False), ((3, 40, 512), 128, True)])
def test_dequant_w4_bit_exact(gpu, shape, gs, frac_zero):
    w4 = load_mod("w4a16")
    g = torch.Generator().manual_seed(sum(shape) + gs)
    lead, K = shape[:-1], shape[-1]
    q = torch.randint(0, 256, lead + (K // 2,), generator=g, dtype=torch.uint8)
    s = (0.005 + 0.015 * torch.rand(lead + (K // gs,), generator=g)).to(torch.float16)
    z = torch.randint(0, 16, lead + (K // gs,), generator=g).to(torch.float16)
    if frac_zero:  # the reference's expression takes any fp16 zero-point
        z = (z + 0.37 * torch.rand(z.shape, generator=g)).to(torch.float16)
    print(f"ksl_dequant_w4 shape={shape} gs={gs} frac_zero={frac_zero}", flush=True)
    W = w4.dequant_w4(q.to(gpu), s.to(gpu), z.to(gpu), gs)
    torch.cuda.synchronize()
    ref = mo.dequant_w4(q.numpy(), s.numpy(), z.numpy(), gs)
    assert W.shape == lead + (K,) and W.dtype == torch.float16
    assert np.array_equal(_np(W).view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("E,H,I", [(3, 2816, 704), (2, 128, 64), (1, 192, 1024)])
def test_preshuffle_T_dn_bytes_and_round_trip(gpu, E, H, I):
    v2 = load_mod("fused_moe_w4_v2")
    g = torch.Generator().manual_seed(E * H + I)
    dn = torch.randint(0, 256, (E, H, I // 2), generator=g, dtype=torch.uint8)
    ns = v2.preshuffle_T_dn(dn.to(gpu))
    back = v2.unshuffle_ns_down(ns)
    torch.cuda.synchronize()
    assert tuple(ns.shape) == (E, I // 2, H)
    assert np.array_equal(_np(ns), mo.preshuffle_ns_down(dn.numpy()))
    assert torch.equal(back.cpu(), dn)


def test_enable_ns_down_gives_the_plain_pack_bits(gpu):
    v2 = load_mod("fused_moe_w4_v2")
    wl = load_mod("workloads")
    T, tk, E, H, I = 64, 8, 16, 512, 704
    ids, w = wl.make_routing(T, E, tk, 101)
    hidden = wl.make_hidden(T, H, 102).to(gpu)
    idsg, wg = ids.to(gpu), w.to(gpu)
    plain = wl.make_experts(E, H, I, 100, act="silu").to(gpu)
    y_plain = v2.fused_moe_w4_v2(hidden, plain, idsg, wg)
    # the reference's load-time switch
    a = wl.make_experts(E, H, I, 100, act="silu").to(gpu)
    assert v2.enable_ns_down(a) is a and a.dn_tiled and not a.dn_ns
    y_a = v2.fused_moe_w4_v2(hidden, a, idsg, wg)
    # a module that arrives as an NS pack (made by the reference's own enable_ns_down)
    b = wl.make_experts(E, H, I, 100, act="silu").to(gpu)
    b.dn_q = v2.preshuffle_T_dn(b.dn_q)
    b.dn_ns = True
    y_b = v2.fused_moe_w4_v2(hidden, b, idsg, wg)
    torch.cuda.synchronize()
    assert b.dn_tiled and not b.dn_ns
    assert torch.equal(y_a.view(torch.int16), y_plain.view(torch.int16))
    assert torch.equal(y_b.view(torch.int16), y_plain.view(torch.int16))


@pytest.mark.parametrize("flag,act,path", [("0", "relu_sq", "v1"), ("1", "silu", "v2"), (None, "silu", "v2"),
                                           (None, "relu_sq", "v1"), ("0", "silu", "v1")])
def test_fused_experts_forward_moe_v2_dispatch(gpu, monkeypatch, flag, act, path):
    """MOE_V2 == "1": the v2 forward; any other value: the v1 forward; unset:
    v2 for an activation the v2 epilogue has, else v1. The v1 result with
    relu^2 is checked against the oracle's moe_forward_v1."""
    pe = load_mod("pack_experts")
    v1 = load_mod("fused_moe_w4")
    v2 = load_mod("fused_moe_w4_v2")
    wl = load_mod("workloads")
    T, tk, E, H, I = 96, 8, 32, 512, 192
    exp = wl.make_experts(E, H, I, 110, act="silu")
    if act == "relu_sq":
        exp.act_fn = _relu_sq
    ids, w = wl.make_routing(T, E, tk, 111)
    hidden = wl.make_hidden(T, H, 112)
    expg, hg, idsg, wg = exp.to(gpu), hidden.to(gpu), ids.to(gpu), w.to(gpu)
    if flag is None:
        monkeypatch.delenv("MOE_V2", raising=False)
    else:
        monkeypatch.setenv("MOE_V2", flag)
    monkeypatch.delenv("MOE_STATS", raising=False)
    y = pe.fused_experts_forward(expg, hg, idsg, wg)
    y_path = (v2.fused_moe_w4_v2 if path == "v2" else v1.fused_moe_w4)(hg, expg, idsg, wg)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_path.view(torch.int16))
    if act == "relu_sq":
        def act16(gate):
            return _relu_sq(torch.from_numpy(gate).float()).half().numpy()
        ref = mo.moe_forward_v1(hidden.float().numpy(), *_experts_np(exp), ids.numpy(), w.float().numpy(), act16)
        ref_b = mo.bf16_to_f32(mo.f32_to_bf16(ref.astype(np.float32)))
        check_norm_err("forward_v1", y.float().cpu().numpy(), ref_b, f"MOE_V2={flag} relu_sq")


def test_moe_stats_probe(gpu, monkeypatch):
    """MOE_STATS=1 records, per forward, the expert union of the top-8/6/4/2
    (by weight) and the experts holding 80% of the routing mass
    (kernels/pack_experts.py:69-78); dump_moe_stats prints their means."""
    pe = load_mod("pack_experts")
    wl = load_mod("workloads")
    T, tk, E, H, I = 64, 8, 32, 256, 128
    exp = wl.make_experts(E, H, I, 120, act="silu").to(gpu)
    ids, w = wl.make_routing(T, E, tk, 121, 1.5)
    hidden = wl.make_hidden(T, H, 122).to(gpu)
    monkeypatch.setenv("MOE_STATS", "1")
    monkeypatch.setenv("MOE_V2", "1")
    pe._MOE_ACC.clear()
    pe.fused_experts_forward(exp, hidden, ids.to(gpu), w.to(gpu))
    pe.fused_experts_forward(exp, hidden, ids.to(gpu), w.to(gpu))
    idn, wn = ids.numpy(), w.numpy()
    order = np.argsort(-wn, axis=-1, kind="stable")
    tis = np.take_along_axis(idn, order, -1)
    for k, key in ((8, "u8"), (6, "u6"), (4, "u4"), (2, "u2")):
        assert pe._MOE_ACC[key] == [len(np.unique(tis[:, :k]))] * 2
    hist = np.sort(np.bincount(idn.reshape(-1), minlength=E))[::-1].astype(np.float64)
    conc = int((np.cumsum(hist) / hist.sum() < 0.8).sum()) + 1
    assert pe._MOE_ACC["conc"] == [conc] * 2 and pe._MOE_ACC["E"] == [E] * 2
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        pe.dump_moe_stats()
    assert "MoE ROUTING PROBE (n=2" in buf.getvalue() and f"of {E}" in buf.getvalue()
    pe._MOE_ACC.clear()


@pytest.mark.parametrize("wdt,ydt", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                     (torch.float16, torch.float16), (torch.float32, torch.float32)])
def test_combine_stock_bit_exact(gpu, wdt, ydt):
    lib = load_pkg()._lib
    wl = load_mod("workloads")
    T, tk, E, H = 256, 8, 128, 2816
    ids, w = wl.make_routing(T, E, tk, 130)
    g = torch.Generator().manual_seed(131)
    out3 = (3 * torch.randn(T * tk, H, generator=g)).to(torch.float16)
    inv = torch.from_numpy(mo.moe_align(ids.numpy(), 1, E)[3].astype(np.int32))
    w = w.to(wdt)
    y = torch.empty(T, H, dtype=ydt, device=gpu)
    o3g, invg, idsg, wg = out3.to(gpu), inv.to(gpu), ids.to(gpu), w.to(gpu)
    lib.check(lib.load().ksl_moe_combine_stock(lib.ptr(o3g), lib.ptr(invg), lib.ptr(idsg), E, lib.ptr(wg),
                                               lib.dtype_code(wdt), T, tk, H, lib.ptr(y), lib.dtype_code(ydt), H,
                                               lib.stream_of(y)), "ksl_moe_combine_stock")
    torch.cuda.synchronize()
    wn = w.float().numpy() if wdt != torch.float16 else w.numpy()
    out = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[ydt]
    ref = mo.combine_stock(out3.numpy(), inv.numpy(), ids.numpy(), wn, E, out)
    got = _np(y.view(torch.int16)).view(np.uint16) if ydt == torch.bfloat16 else _np(y)
    if ydt == torch.bfloat16:
        assert np.array_equal(got, ref)
    else:
        assert np.array_equal(got.view(np.uint8), np.asarray(ref).view(np.uint8))


class _Experts(torch.nn.Module):
    """A bf16 experts module as the model holds it before packing."""

    def __init__(self, E, H, I, seed, act):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.gate_up_proj = torch.nn.Parameter((0.02 * torch.randn(E, 2 * I, H, generator=g)).to(torch.bfloat16),
                                               requires_grad=False)
        self.down_proj = torch.nn.Parameter((0.02 * torch.randn(E, H, I, generator=g)).to(torch.bfloat16),
                                            requires_grad=False)
        self.act_fn = act


@pytest.mark.parametrize("act", ["gelu", "relu_sq"])
def test_packed_experts_forward_matches_the_oracle(gpu, act):
    """pack_experts_module(exp, True, False) binds the packed loop; its output
    is the oracle's stock-loop forward within the v1 bar, rerun bit-identical."""
    pe = load_mod("pack_experts")
    wl = load_mod("workloads")
    fn = wl.gelu_pytorch_tanh if act == "gelu" else _relu_sq
    E, H, I, T, tk = 16, 512, 192, 64, 8
    exp = _Experts(E, H, I, 140, fn).to(gpu)
    pe.pack_experts_module(exp, True, False)
    assert exp.forward.__func__ is pe.packed_experts_forward
    ids, w = wl.make_routing(T, E, tk, 141)
    hidden = wl.make_hidden(T, H, 142)
    y = exp(hidden.to(gpu), ids.to(gpu), w.to(gpu))
    y2 = exp(hidden.to(gpu), ids.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    assert y.dtype == hidden.dtype and torch.equal(y.view(torch.int16), y2.view(torch.int16))
    qs = _experts_np(exp)
    qs[3] = mo.untile_down(qs[3], I)

    def act16(gate):
        return fn(torch.from_numpy(gate).float()).half().numpy()

    ref = mo.moe_forward_stock(hidden.float().numpy(), *qs, ids.numpy(), w.float().numpy(), act16, "bf16")
    check_norm_err("forward_v1", y.float().cpu().numpy(), mo.bf16_to_f32(ref), f"packed loop {act}")
    # the default binds the fused forward, as the reference's fused=True
    other = _Experts(E, H, I, 143, fn).to(gpu)
    pe.pack_experts_module(other)
    assert other.forward.__func__ is pe.fused_experts_forward


def test_repack_cache_binds_only_a_modules_own_weights(gpu):
    """One cache across modules: module a's original dn_q is freed once a is
    repacked, and module b's dn_q (same size) may be allocated at the freed
    address. b must still get its own tiled weights (the cache entry keeps a
    weak reference to its source and is used only for that very tensor)."""
    v2 = load_mod("fused_moe_w4_v2")
    wl = load_mod("workloads")
    T, tk, E, H, I = 32, 4, 8, 256, 192
    ids, w = wl.make_routing(T, E, tk, 151)
    hidden = wl.make_hidden(T, H, 152).to(gpu)
    idsg, wg = ids.to(gpu), w.to(gpu)
    cache: dict = {}
    a = wl.make_experts(E, H, I, 153, act="silu").to(gpu)
    a_ptr = a.dn_q.data_ptr()
    v2.enable_tiled_down(a, cache)
    v2.enable_pack(a, cache)
    torch.cuda.synchronize()
    b_cpu = wl.make_experts(E, H, I, 154, act="silu")
    b = b_cpu.to(gpu)
    print(f"dn_q address reused: {b.dn_q.data_ptr() == a_ptr}", flush=True)
    b_plain = b_cpu.to(gpu)
    y_ref = v2.fused_moe_w4_v2(hidden, b_plain, idsg, wg)
    v2.enable_tiled_down(b, cache)
    v2.enable_pack(b, cache)
    assert b.dn_q.data_ptr() != a.dn_q.data_ptr() and b.gu_pack.data_ptr() != a.gu_pack.data_ptr()
    y_b = v2.fused_moe_w4_v2(hidden, b, idsg, wg)
    torch.cuda.synchronize()
    assert torch.equal(y_b.view(torch.int16), y_ref.view(torch.int16))
