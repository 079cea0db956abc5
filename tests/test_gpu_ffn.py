"""GPU parity of the one-launch expert FFN (ksl_moe_ffn) and its load-time
pack (ksl_moe_pack_gateup / ksl_moe_pack_down), through the C ABI.

Bars:
- the pack: read back by the oracle (oracle/moe_oracle.py unpack_gateup /
  unpack_down), it is the reference buffers byte for byte, from both down
  layouts;
- out2 and out3 of the one launch are bit-identical to the gate/up and down
  launches on the reference layout (whose parity against the oracle is
  tests/test_gpu_moe.py's), on every routed row; the whole forward through the
  drop-in is bit-identical with and without the pack;
- the counters are left zero after every launch (a second launch on the same
  counters gives the same bits) and the bounded-wait error word stays 0.
Cases cover multi-chunk experts (more than 32 rows), experts without rows,
narrow last units (I % 176 != 0, H % 352 != 0), I with and without a 64-K
tail, fewer 128-K groups than ring slots, and 8192 routed rows.
"""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from tests._helpers import bf16_bits, check_norm_err
from tests.conftest import load_mod, load_pkg

pytestmark = pytest.mark.gpu

CTL_STRIDE = 64  # int32 words between two counters of the ctl array (slot 1: the error word)

FFN_CASES = [
    # (T, tk, E, H, I, seed, zipf)
    (256, 8, 128, 2816, 704, 61, None),   # the layer_256 canvas
    (64, 8, 16, 512, 192, 62, None),      # narrow last units of gate/up (1 tile) and down (10 tiles), 64-K tail
    (48, 4, 8, 384, 704, 63, None),       # 3 groups of 128 K (as many as the early-issued slots)
    (16, 2, 4, 256, 128, 64, None),       # 2 groups: fewer than the ring's early slots, no tail
    (512, 8, 16, 256, 256, 65, None),     # 256 rows per expert: 8 chunks of 32
    (64, 2, 64, 256, 704, 66, 1.5),       # skewed: experts without rows, heavy ones
    (1024, 8, 128, 2816, 704, 67, None),  # 8192 routed rows (the largest the one launch takes)
    (64, 4, 8, 256, 1024, 68, None),      # I = 1024: 8 groups of 128, no tail
]


def _route(gpu, ids, hidden, E):
    lib = load_pkg()._lib
    T, tk = ids.shape
    H = hidden.shape[1]
    sr = torch.empty(T * tk, dtype=torch.int32, device=gpu)
    off = torch.empty(E + 1, dtype=torch.int32, device=gpu)
    inv = torch.empty(T * tk, dtype=torch.int32, device=gpu)
    a16 = torch.empty(T, H, dtype=torch.float16, device=gpu)
    rc = lib.load().ksl_moe_route(lib.ptr(ids), T, tk, E, lib.ptr(sr), lib.ptr(off), lib.ptr(inv),
                                  lib.ptr(hidden), lib.dtype_code(hidden.dtype), hidden.stride(0), H,
                                  lib.ptr(a16), lib.stream_of(ids))
    lib.check(rc, "ksl_moe_route")
    return sr, off, inv, a16


def _pack(gpu, exp, dn_layout):
    lib = load_pkg()._lib
    L = lib.load()
    E, twoI, Hh = exp.gu_q.shape
    H, I = 2 * Hh, twoI // 2
    gu = torch.empty(int(L.ksl_moe_pack_gateup_bytes(E, H, I)), dtype=torch.uint8, device=gpu)
    dn = torch.empty(int(L.ksl_moe_pack_down_bytes(E, H, I)), dtype=torch.uint8, device=gpu)
    st = lib.stream_of(gu)
    lib.check(L.ksl_moe_pack_gateup(lib.ptr(exp.gu_q), lib.ptr(exp.gu_s), lib.ptr(exp.gu_z), E, H, I, lib.ptr(gu),
                                    st), "ksl_moe_pack_gateup")
    dq = exp.dn_q
    if dn_layout == lib.DN_LAYOUT_TILED:
        dq = load_mod("fused_moe_w4_v2").tiled_down(exp.dn_q, exp.dn_s, exp.dn_z)
    lib.check(L.ksl_moe_pack_down(lib.ptr(dq), lib.ptr(exp.dn_s), lib.ptr(exp.dn_z), dn_layout, E, H, I,
                                  lib.ptr(dn), st), "ksl_moe_pack_down")
    return gu, dn


@pytest.mark.parametrize("E,H,I", [(3, 384, 704), (2, 512, 192), (2, 256, 1024), (1, 2816, 704)])
@pytest.mark.parametrize("tiled", [False, True])
def test_pack_reads_back_to_the_reference_buffers(gpu, E, H, I, tiled):
    lib = load_pkg()._lib
    wl = load_mod("workloads")
    exp = wl.make_experts(E, H, I, 70 + E).to(gpu)
    gu, dn = _pack(gpu, exp, lib.DN_LAYOUT_TILED if tiled else lib.DN_LAYOUT_REF)
    torch.cuda.synchronize()
    q, s, z = mo.unpack_gateup(gu.cpu().numpy(), E, H, I)
    assert np.array_equal(q, exp.gu_q.cpu().numpy())
    assert np.array_equal(s.view(np.uint16), exp.gu_s.cpu().numpy().view(np.uint16))
    assert np.array_equal(z.view(np.uint16), exp.gu_z.cpu().numpy().view(np.uint16))
    q, s, z = mo.unpack_down(dn.cpu().numpy(), E, H, I)
    assert np.array_equal(q, exp.dn_q.cpu().numpy())
    assert np.array_equal(s.view(np.uint16), exp.dn_s.cpu().numpy().view(np.uint16))
    assert np.array_equal(z.view(np.uint16), exp.dn_z.cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("T,tk,E,H,I,seed,zipf", FFN_CASES)
def test_ffn_bit_identical_to_gateup_and_down(gpu, act, T, tk, E, H, I, seed, zipf):
    lib = load_pkg()._lib
    L = lib.load()
    wl = load_mod("workloads")
    code = lib.ACT_SILU if act == "silu" else lib.ACT_GELU_TANH
    exp = wl.make_experts(E, H, I, seed, act=act).to(gpu)
    ids, _ = wl.make_routing(T, E, tk, seed + 1, zipf)
    hidden = wl.make_hidden(T, H, seed + 2).to(gpu)
    idsg = ids.to(gpu)
    nexp = T * tk
    sr, off, inv, a16 = _route(gpu, idsg, hidden, E)
    st = lib.stream_of(hidden)
    # the two-launch stages on the reference layout
    out2_ref = torch.empty(nexp, I, dtype=torch.float16, device=gpu)
    out3_ref = torch.empty(nexp, H, dtype=torch.float16, device=gpu)
    lib.check(L.ksl_moe_gateup_act(lib.ptr(a16), lib.ptr(sr), lib.ptr(off), T, tk, lib.ptr(exp.gu_q),
                                   lib.ptr(exp.gu_s), lib.ptr(exp.gu_z), E, H, I, code, lib.ptr(out2_ref), st),
              "ksl_moe_gateup_act")
    lib.check(L.ksl_moe_down(lib.ptr(out2_ref), lib.ptr(off), lib.ptr(exp.dn_q), lib.ptr(exp.dn_s),
                             lib.ptr(exp.dn_z), E, H, I, nexp, lib.ptr(out3_ref), lib.DN_LAYOUT_REF, st),
              "ksl_moe_down")
    # the one launch on the pack, twice on the same counters
    gu, dn = _pack(gpu, exp, lib.DN_LAYOUT_REF)
    ctl = torch.zeros(int(L.ksl_moe_ffn_ctl_bytes(E)) // 4, dtype=torch.int32, device=gpu)
    outs = []
    for rep in range(2):
        out2 = torch.full((nexp, I), float("nan"), dtype=torch.float16, device=gpu)
        out3 = torch.full((nexp, H), float("nan"), dtype=torch.float16, device=gpu)
        print(f"ksl_moe_ffn {act} T={T} tk={tk} E={E} H={H} I={I} zipf={zipf} call {rep}", flush=True)
        lib.check(L.ksl_moe_ffn(lib.ptr(a16), lib.ptr(sr), lib.ptr(off), T, tk, lib.ptr(gu), lib.ptr(dn), E, H, I,
                                code, lib.ptr(out2), lib.ptr(out3), lib.ptr(ctl), st), "ksl_moe_ffn")
        torch.cuda.synchronize()
        outs.append((out2, out3))
        c = ctl.cpu().numpy()
        assert c[CTL_STRIDE * 1] == 0, "a wait for another workgroup ran out of its bound"
        assert not c.any(), f"counters not cleared: {np.nonzero(c)[0][:8]}"
    nrows = int(off[E].item())
    counts = np.diff(off.cpu().numpy())
    print(f"routed rows {nrows}, rows per expert {counts.min()}..{counts.max()}, "
          f"experts without rows {(counts == 0).sum()}", flush=True)
    for out2, out3 in outs:
        assert torch.equal(out2[:nrows].view(torch.int16), out2_ref[:nrows].view(torch.int16))
        assert torch.equal(out3[:nrows].view(torch.int16), out3_ref[:nrows].view(torch.int16))


def test_drop_in_forward_same_with_and_without_pack(gpu):
    """fused_moe_w4_v2 and moe_layer give the same bits whether the experts
    carry the pack (one launch) or not (gate/up + down), and stay within the
    oracle's tolerance."""
    pkg = load_pkg()
    v2 = load_mod("fused_moe_w4_v2")
    layer = load_mod("layer")
    wl = load_mod("workloads")
    T, tk, E, H, I = 96, 8, 32, 512, 704
    exp = wl.make_experts(E, H, I, 80, act="silu").to(gpu)
    x, nw, ids, w = wl.layer_inputs(T, 81, E=E, k=tk, H=H)
    xg, nwg, idsg, wg = x.to(gpu), nw.to(gpu), ids.to(gpu), w.to(gpu)
    hidden = pkg.fused_rmsnorm(xg, nwg, 1e-6)
    y0 = v2.fused_moe_w4_v2(hidden, exp, idsg, wg)
    l0 = layer.moe_layer(xg, nwg, 1e-6, exp, idsg, wg)
    v2.enable_pack(exp)
    assert exp.gu_pack is not None and exp.dn_pack is not None
    y1 = v2.fused_moe_w4_v2(hidden, exp, idsg, wg)
    l1 = layer.moe_layer(xg, nwg, 1e-6, exp, idsg, wg)
    v2.enable_tiled_down(exp)  # the pack survives the down repack
    l2 = layer.moe_layer(xg, nwg, 1e-6, exp, idsg, wg)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(l0.view(torch.int16), l1.view(torch.int16))
    assert torch.equal(l0.view(torch.int16), l2.view(torch.int16))
    qs = [getattr(exp, k).cpu().numpy() for k in ("gu_q", "gu_s", "gu_z")]
    dn_q = mo.untile_down(exp.dn_q.cpu().numpy(), I)
    ref, _, _ = mo.moe_forward_per_expert(hidden.float().cpu().numpy(), *qs, dn_q, exp.dn_s.cpu().numpy(),
                                          exp.dn_z.cpu().numpy(), ids.numpy(), w.numpy(), mo.ACT_SILU)
    check_norm_err("ffn_dropin", y1.float().cpu().numpy(), ref, "fused_moe_w4_v2 with the pack")


def test_layer_runner_ffn_stages_match_the_fused_call(gpu):
    """LayerRunner's one-launch stages (route + RMSNorm, ffn, combine) give the
    bits of the fused call, on the layer_256 shapes."""
    v2 = load_mod("fused_moe_w4_v2")
    layer = load_mod("layer")
    wl = load_mod("workloads")
    T, tk, E, H, I = 256, 8, 128, 2816, 704
    exp = wl.make_experts(E, H, I, 90, act="silu").to(gpu)
    v2.enable_pack(exp)
    x, nw, ids, w = wl.layer_inputs(T, 91)
    xg, nwg, idsg, wg = x.to(gpu), nw.to(gpu), ids.to(gpu), w.to(gpu)
    y = layer.moe_layer(xg, nwg, 1e-6, exp, idsg, wg)
    runner = layer.LayerRunner(T, tk, E, H, I, gpu)
    assert runner.stages(exp) == layer.STAGES_FFN
    ys = [runner.run(xg, nwg, 1e-6, exp, idsg, wg).clone() for _ in range(3)]
    # int32 ids and a non-contiguous weight view are converted, not misread
    ys.append(runner.run(xg, nwg, 1e-6, exp, idsg.to(torch.int32), wg.t().contiguous().t()).clone())
    torch.cuda.synchronize()
    for r in ys:
        assert np.array_equal(bf16_bits(r), bf16_bits(y))


def test_failed_wait_poisons_the_call(gpu):
    """A down unit whose bounded wait for its expert's gate/up units gives up
    sets the error word, and the fused forwards then return NaN for that call
    instead of normal-looking output. The failure is forced from the host
    (every dependency counts as unmet, a bound of 4 empty ring cycles): each
    down unit waits out the bound and runs, every workgroup finishes normally.
    The next call with the default bound is clean and equals the first."""
    lib = load_pkg()._lib
    L = lib.load()
    v2 = load_mod("fused_moe_w4_v2")
    layer = load_mod("layer")
    pkg = load_pkg()
    wl = load_mod("workloads")
    T, tk, E, H, I = 64, 8, 16, 512, 192
    exp = wl.make_experts(E, H, I, 95, act="silu").to(gpu)
    v2.enable_pack(exp)
    x, nw, ids, w = wl.layer_inputs(T, 96, E=E, k=tk, H=H)
    xg, nwg, idsg, wg = x.to(gpu), nw.to(gpu), ids.to(gpu), w.to(gpu)
    hidden = pkg.fused_rmsnorm(xg, nwg, 1e-6)
    y_ok = layer.moe_layer(xg, nwg, 1e-6, exp, idsg, wg)
    f_ok = v2.fused_moe_w4_v2(hidden, exp, idsg, wg)
    torch.cuda.synchronize()
    assert not torch.isnan(y_ok).any() and not torch.isnan(f_ok).any()
    runner = layer.LayerRunner(T, tk, E, H, I, gpu)
    lib.check(L.ksl_moe_ffn_set_wait_limit(4, 1), "ksl_moe_ffn_set_wait_limit")
    try:
        print(f"forced failed wait: moe_layer / fused_moe_w4_v2 / LayerRunner T={T} E={E} H={H} I={I}", flush=True)
        y_bad = layer.moe_layer(xg, nwg, 1e-6, exp, idsg, wg)
        f_bad = v2.fused_moe_w4_v2(hidden, exp, idsg, wg)
        runner.run(xg, nwg, 1e-6, exp, idsg, wg)
        torch.cuda.synchronize()
    finally:
        lib.check(L.ksl_moe_ffn_set_wait_limit(-1, 0), "ksl_moe_ffn_set_wait_limit")
    assert torch.isnan(y_bad).all(), "moe_layer returned normal-looking output after a failed wait"
    assert torch.isnan(f_bad).all(), "fused_moe_w4_v2 returned normal-looking output after a failed wait"
    # the standalone launch latches the error word in the caller's counters
    assert runner.ffn_error(), "the runner's error word was not set"
    c = runner.ctl.cpu().numpy()
    c[CTL_STRIDE * 1] = 0
    assert not c.any(), "counters other than the error word not cleared"
    # a normal call afterwards: the routing clears the word, same bits as before
    y_again = layer.moe_layer(xg, nwg, 1e-6, exp, idsg, wg)
    torch.cuda.synchronize()
    assert torch.equal(y_again.view(torch.int16), y_ok.view(torch.int16))
    # out-of-range bounds are refused
    assert L.ksl_moe_ffn_set_wait_limit(1 << 31, 0) == lib.ERR_ARG
