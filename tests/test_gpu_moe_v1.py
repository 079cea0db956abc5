"""GPU parity for the reference's v1 MoE path (kernels/fused_moe_w4.py:54-128):
the gate/up GEMM without activation, the activation reorder, the v1 combine
and the whole fused_moe_w4 with a generic act_fn, through the C ABI.

Bars:
- activation reorder and v1 combine (integer / rounding work): bit-exact vs
  the oracle on the same inputs;
- gate/up without activation and the forward (floating point): normalised
  max / mean error within BARS["gateup_raw"] / BARS["forward_v1"], about
  twice the values observed on the MI355X (printed in the terminal summary).
"""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from tests._helpers import check_norm_err, f16_bits, out2_unperm
from tests.conftest import load_mod, load_pkg

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _experts_np(exp):
    return [_np(getattr(exp, k)) for k in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z")]


@pytest.mark.parametrize("rows,I", [(37, 128), (256, 704), (5, 832), (64, 64), (1, 1024)])
def test_act_to_down_order_bit_exact(gpu, rows, I):
    lib = load_pkg()._lib
    g = torch.Generator().manual_seed(rows * 1000 + I)
    x = torch.randn(rows, I, generator=g).to(torch.float16)
    xg = x.to(gpu)
    out = torch.empty_like(xg)
    lib.check(lib.load().ksl_moe_act_to_down_order(lib.ptr(xg), rows, I, lib.ptr(out), lib.stream_of(xg)),
              "ksl_moe_act_to_down_order")
    torch.cuda.synchronize()
    assert np.array_equal(out2_unperm(f16_bits(out.cpu()), I), f16_bits(x))


@pytest.mark.parametrize("wdt,ydt", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                     (torch.float32, torch.float16), (torch.float16, torch.float32)])
def test_combine_v1_bit_exact(gpu, wdt, ydt):
    lib = load_pkg()._lib
    wl = load_mod("workloads")
    T, tk, E, H = 256, 8, 128, 2816
    ids, w = wl.make_routing(T, E, tk, 61)
    g = torch.Generator().manual_seed(62)
    out3 = (3 * torch.randn(T * tk, H, generator=g)).to(torch.float16)
    ref_inv = mo.moe_align(ids.numpy(), 1, E)[3]
    inv = torch.from_numpy(ref_inv.astype(np.int32))
    w = w.to(wdt)
    y = torch.empty(T, H, dtype=ydt, device=gpu)
    o3g, invg, wg = out3.to(gpu), inv.to(gpu), w.to(gpu)
    lib.check(lib.load().ksl_moe_combine_v1(lib.ptr(o3g), lib.ptr(invg), lib.ptr(wg), lib.dtype_code(wdt), T, tk,
                                            H, lib.ptr(y), lib.dtype_code(ydt), H, lib.stream_of(y)),
              "ksl_moe_combine_v1")
    ref = torch.from_numpy(mo.combine_v1(out3.numpy(), ref_inv, w.float().numpy())).to(ydt)
    assert torch.equal(y.cpu().view(torch.uint8), ref.view(torch.uint8))


def _route(gpu, ids, hidden, E):
    lib = load_pkg()._lib
    T, tk = ids.shape
    H = hidden.shape[1]
    sr = torch.empty(T * tk, dtype=torch.int32, device=gpu)
    off = torch.empty(E + 1, dtype=torch.int32, device=gpu)
    inv = torch.empty(T * tk, dtype=torch.int32, device=gpu)
    a16 = torch.empty(T, H, dtype=torch.float16, device=gpu)
    lib.check(lib.load().ksl_moe_route(lib.ptr(ids), T, tk, E, lib.ptr(sr), lib.ptr(off), lib.ptr(inv),
                                       lib.ptr(hidden), lib.dtype_code(hidden.dtype), hidden.stride(0), H,
                                       lib.ptr(a16), lib.stream_of(ids)), "ksl_moe_route")
    return sr, off, inv, a16


GU_RAW_CASES = [
    # (T, tk, E, H, I, seed): 64-, 128- and 176-column blocks, the layer's shape,
    # above 8192 routed rows (still the per-expert kernel without activation)
    (16, 2, 4, 256, 64, 71),
    (40, 4, 4, 640, 128, 72),
    (256, 8, 128, 2816, 704, 73),
    (1100, 8, 12, 256, 704, 74),
]


@pytest.mark.parametrize("T,tk,E,H,I,seed", GU_RAW_CASES)
def test_gateup_without_activation(gpu, T, tk, E, H, I, seed):
    lib = load_pkg()._lib
    wl = load_mod("workloads")
    exp = wl.make_experts(E, H, I, seed).to(gpu)
    ids, _ = wl.make_routing(T, E, tk, seed + 1)
    hidden = wl.make_hidden(T, H, seed + 2)
    sr, off, inv, a16 = _route(gpu, ids.to(gpu), hidden.to(gpu), E)
    out1 = torch.empty(T * tk, 2 * I, dtype=torch.float16, device=gpu)
    lib.check(lib.load().ksl_moe_gateup_act(lib.ptr(a16), lib.ptr(sr), lib.ptr(off), T, tk, lib.ptr(exp.gu_q),
                                            lib.ptr(exp.gu_s), lib.ptr(exp.gu_z), E, H, I, lib.ACT_NONE,
                                            lib.ptr(out1), lib.stream_of(a16)), "ksl_moe_gateup_act")
    got = _np(out1)[_np(inv).astype(np.int64)].astype(np.float32)  # expanded-row order
    gu_q, gu_s, gu_z = (_np(exp.gu_q), _np(exp.gu_s), _np(exp.gu_z))
    flat = ids.numpy().reshape(-1)
    a = hidden.float().numpy().astype(np.float16)
    ref = np.zeros((T * tk, 2 * I), np.float32)
    for e in range(E):
        r = np.nonzero(flat == e)[0]
        if r.size:
            ref[r] = mo.gateup_raw(a[r // tk], mo.dequant_w4(gu_q[e], gu_s[e], gu_z[e], mo.GU_GS))
    check_norm_err("gateup_raw", got, ref, f"T={T} E={E} H={H} I={I}")


def _relu_sq(x):
    return torch.relu(x) ** 2


V1_CASES = [
    # (T, tk, E, H, I, seed, act): tanh-GELU as the reference's v1 runs it, and
    # activations the v2 epilogue does not have
    (64, 8, 16, 512, 192, 81, "gelu"),
    (256, 8, 128, 2816, 704, 82, "gelu"),
    (256, 8, 128, 2816, 704, 83, "relu_sq"),
    (48, 4, 8, 384, 704, 84, "mish"),
]
_ACT_FNS = {"gelu": load_mod("workloads").gelu_pytorch_tanh, "relu_sq": _relu_sq,
            "mish": torch.nn.functional.mish}


@pytest.mark.parametrize("T,tk,E,H,I,seed,act", V1_CASES)
def test_fused_moe_w4_v1_forward(gpu, T, tk, E, H, I, seed, act):
    v1 = load_mod("fused_moe_w4")
    wl = load_mod("workloads")
    exp = wl.make_experts(E, H, I, seed)
    fn = _ACT_FNS[act]
    exp.act_fn = fn
    ids, w = wl.make_routing(T, E, tk, seed + 1)
    hidden = wl.make_hidden(T, H, seed + 2)
    expg = exp.to(gpu)
    y = v1.fused_moe_w4(hidden.to(gpu), expg, ids.to(gpu), w.to(gpu))
    assert y.dtype == hidden.dtype and y.shape == (T, H)

    def act16(gate):  # the same function on the CPU, computed in fp32 as torch's fp16 GPU ops do
        return fn(torch.from_numpy(gate).float()).half().numpy()

    ref = mo.moe_forward_v1(hidden.float().numpy(), *_experts_np(exp), ids.numpy(), w.float().numpy(), act16)
    ref_b = ref.astype(np.float32)
    if hidden.dtype == torch.bfloat16:
        ref_b = mo.bf16_to_f32(mo.f32_to_bf16(ref_b))
    check_norm_err("forward_v1", y.float().cpu().numpy(), ref_b, f"{act} T={T} E={E} H={H} I={I}")
    y2 = v1.fused_moe_w4(hidden.to(gpu), expg, ids.to(gpu), w.to(gpu))
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))


def test_fused_moe_w4_v1_strided_and_offset_hidden(gpu):
    """A row-strided view, and a view starting 2 bytes into its storage (not
    16-byte aligned): the same bits as the contiguous input (the wrapper copies
    what the routing launch cannot read in place)."""
    v1 = load_mod("fused_moe_w4")
    wl = load_mod("workloads")
    T, tk, E, H, I = 32, 4, 8, 256, 128
    exp = wl.make_experts(E, H, I, 91).to(gpu)
    ids, w = wl.make_routing(T, E, tk, 92)
    hidden = wl.make_hidden(T, H, 93).to(gpu)
    ref = v1.fused_moe_w4(hidden, exp, ids.to(gpu), w.to(gpu))
    wide = torch.zeros(T, H + 24, dtype=hidden.dtype, device=gpu)
    wide[:, :H] = hidden
    y1 = v1.fused_moe_w4(wide[:, :H], exp, ids.to(gpu), w.to(gpu))
    flat = torch.zeros(T * H + 1, dtype=hidden.dtype, device=gpu)
    off = flat[1:].view(T, H)
    off.copy_(hidden)
    y2 = v1.fused_moe_w4(off, exp, ids.to(gpu), w.to(gpu))
    assert torch.equal(ref.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(ref.view(torch.int16), y2.view(torch.int16))
