"""GPU tests of the load-time paths of the MoE weights, through the C ABI.

- The MOE_NS down pack (the reference's preshuffle_T_dn,
  kernels/fused_moe_w4_v2.py:187-197, restated by oracle preshuffle_ns_down,
  which tests/test_cpu_oracle.py pins to the stated byte rule):
  ksl_moe_unshuffle_ns_down inverts it byte for byte, and a module flagged
  dn_ns runs with the plain pack's output bits.
- The zero-point contract is checked at load time (enable_tiled_down) and
  the forward of a module never synchronises the host: its first call can
  be captured into a graph, and every replay equals the eager result.
"""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from tests.conftest import load_mod

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("E,H,I", [(2, 256, 704), (3, 128, 64), (1, 2816, 704), (2, 64, 1024)])
def test_unshuffle_ns_down_inverts_the_reference_preshuffle(gpu, E, H, I):
    v2 = load_mod("fused_moe_w4_v2")
    q = np.random.default_rng(E * H + I).integers(0, 256, size=(E, H, I // 2)).astype(np.uint8)
    ns = mo.preshuffle_ns_down(q)
    print(f"ksl_moe_unshuffle_ns_down E={E} H={H} I={I}", flush=True)
    out = v2.unshuffle_ns_down(torch.from_numpy(ns).to(gpu))
    torch.cuda.synchronize()
    assert out.shape == (E, H, I // 2)
    assert np.array_equal(out.cpu().numpy(), q)


def test_ns_module_gives_the_plain_pack_output(gpu):
    wl = load_mod("workloads")
    v2 = load_mod("fused_moe_w4_v2")
    T, tk, E, H, I = 64, 8, 16, 512, 704
    plain = wl.make_experts(E, H, I, 41).to(gpu)
    ns = wl.make_experts(E, H, I, 41).to(gpu)
    ns.dn_q = torch.from_numpy(mo.preshuffle_ns_down(ns.dn_q.cpu().numpy())).to(gpu)
    ns.dn_ns = True  # what the reference's enable_ns_down leaves (kernels/fused_moe_w4_v2.py:200-206)
    hidden = wl.make_hidden(T, H, 42).to(gpu)
    ids, w = wl.make_routing(T, E, tk, 43)
    ids, w = ids.to(gpu), w.to(gpu)
    y0 = v2.fused_moe_w4_v2(hidden, plain, ids, w)
    y1 = v2.fused_moe_w4_v2(hidden, ns, ids, w)
    torch.cuda.synchronize()
    assert ns.dn_tiled and not ns.dn_ns
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))


def test_zero_points_are_checked_at_load_time(gpu):
    wl = load_mod("workloads")
    v2 = load_mod("fused_moe_w4_v2")
    exp = wl.make_experts(4, 256, 128, 44).to(gpu)
    exp.dn_z[1, 3, 0] = 2.5
    with pytest.raises(ValueError, match="zero-points"):
        v2.enable_tiled_down(exp)
    exp2 = wl.make_experts(4, 256, 128, 45).to(gpu)
    exp2.gu_z[0, 0, 0] = 16.0
    with pytest.raises(ValueError, match="zero-points"):
        v2.enable_pack(exp2)


def test_first_forward_is_capture_safe(gpu):
    """A module's first fused_moe_w4_v2 call, captured: no host sync inside
    (a sync would fail the capture). Replays with eager work between them
    each equal the eager result bit for bit."""
    wl = load_mod("workloads")
    v2 = load_mod("fused_moe_w4_v2")
    T, tk, E, H, I = 32, 8, 16, 256, 192
    hidden = wl.make_hidden(T, H, 46).to(gpu)
    ids, w = wl.make_routing(T, E, tk, 47)
    ids, w = ids.to(gpu), w.to(gpu)
    warm = wl.make_experts(E, H, I, 48).to(gpu)
    v2.fused_moe_w4_v2(hidden, warm, ids, w)  # the library's one-time set-up happens outside the capture
    exp = wl.make_experts(E, H, I, 49).to(gpu)
    ref_exp = wl.make_experts(E, H, I, 49).to(gpu)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = v2.fused_moe_w4_v2(hidden, exp, ids, w)  # exp's first call
    ref = v2.fused_moe_w4_v2(hidden, ref_exp, ids, w)
    torch.cuda.synchronize()
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"replay {rep}"
        v2.fused_moe_w4_v2(hidden, warm, ids, w)  # eager work between replays
        torch.cuda.synchronize()
