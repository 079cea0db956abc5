"""ksl_moe_layer_forward_noalloc, the layer forward on the library's own
per-GPU scratch array, through the C ABI: the same bits as
ksl_moe_layer_forward on a caller workspace, on two calls in a row (the
second smaller, so it runs on what the first left in the array), over the
two-launch path and the one-launch expert FFN (whose counters then live in
the array); and shapes past KSL_NOALLOC_SCRATCH_BYTES are refused before any
device work."""
import numpy as np
import pytest
import torch

from tests._helpers import bf16_bits
from tests.conftest import load_mod, load_pkg

pytestmark = pytest.mark.gpu


def _forward(L, lib, fn, xg, nwg, idsg, wg, exp, T, tk, E, H, I, y, ws=None):
    st = lib.stream_of(xg)
    args = [lib.ptr(xg), lib.DTYPE_BF16, H, lib.ptr(nwg), lib.DTYPE_BF16, 1e-6, lib.ptr(idsg), lib.ptr(wg),
            lib.DTYPE_F32, lib.ptr(exp.gu_q), lib.ptr(exp.gu_s), lib.ptr(exp.gu_z), lib.ptr(exp.dn_q),
            lib.ptr(exp.dn_s), lib.ptr(exp.dn_z), load_mod("fused_moe_w4_v2").dn_layout(exp),
            *load_mod("fused_moe_w4_v2").pack_ptrs(exp), T, tk, E, H, I, exp._ksl_act, lib.ptr(y),
            lib.DTYPE_BF16, H]
    if ws is not None:
        args += [lib.ptr(ws), ws.numel()]
    return fn(*args, st)


@pytest.mark.parametrize("pack", [False, True])
def test_noalloc_matches_the_workspace_forward(gpu, pack):
    pkg = load_pkg()
    lib = pkg._lib
    L = lib.load()
    v2 = load_mod("fused_moe_w4_v2")
    wl = load_mod("workloads")
    tk, E, H, I = 8, 128, 2816, 704
    exp = wl.make_experts(E, H, I, 100, act="silu").to(gpu)
    v2._check_act(exp)
    v2.enable_tiled_down(exp)
    if pack:
        v2.enable_pack(exp)
    for T, seed in ((256, 101), (40, 102)):  # the second call is smaller
        x, nw, ids, w = wl.layer_inputs(T, seed, E=E, k=tk, H=H)
        xg, nwg, idsg, wg = x.to(gpu), nw.to(gpu), ids.to(gpu), w.to(gpu)
        ws = v2.moe_workspace(T, tk, E, H, I, gpu)
        y_ws = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
        y_na = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=gpu)
        print(f"layer forward pack={pack} T={T}: workspace, then no-alloc", flush=True)
        lib.check(_forward(L, lib, L.ksl_moe_layer_forward, xg, nwg, idsg, wg, exp, T, tk, E, H, I, y_ws, ws),
                  "ksl_moe_layer_forward")
        lib.check(_forward(L, lib, L.ksl_moe_layer_forward_noalloc, xg, nwg, idsg, wg, exp, T, tk, E, H, I, y_na),
                  "ksl_moe_layer_forward_noalloc")
        torch.cuda.synchronize()
        assert np.array_equal(bf16_bits(y_na), bf16_bits(y_ws)), f"T={T}"


def test_noalloc_refuses_shapes_past_its_scratch(gpu):
    lib = load_pkg()._lib
    L = lib.load()
    tk, E, H, I = 8, 128, 2816, 704
    T = 1024  # needs about 64 MB of workspace
    need = int(L.ksl_moe_workspace_bytes(T, tk, E, H, I))
    assert need > lib.NOALLOC_SCRATCH_BYTES
    y = torch.empty(1, dtype=torch.bfloat16, device=gpu)
    # every device pointer is a dummy: the size check returns before any device work
    d = lib.ptr(y)
    rc = L.ksl_moe_layer_forward_noalloc(d, lib.DTYPE_BF16, H, d, lib.DTYPE_BF16, 1e-6, d, d, lib.DTYPE_F32, d, d, d,
                                         d, d, d, lib.DN_LAYOUT_REF, None, None, T, tk, E, H, I, lib.ACT_SILU, d,
                                         lib.DTYPE_BF16, H, lib.stream_of(y))
    assert rc == lib.ERR_SCRATCH
    assert "scratch" in L.ksl_status_string(rc).decode()
