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


def test_ns_modules_sharing_a_buffer_share_the_converted_one(gpu):
    """Encoder and decoder experts of a layer share their buffers
    (kernels/load_w4_checkpoint.py:56-59). Two modules flagged dn_ns over one
    dn_q, converted at their first forwards (no load-time repack ran), end up
    on one converted tensor, with the plain pack's output bits."""
    wl = load_mod("workloads")
    v2 = load_mod("fused_moe_w4_v2")
    T, tk, E, H, I = 32, 8, 16, 256, 704
    plain = wl.make_experts(E, H, I, 61).to(gpu)
    enc = wl.make_experts(E, H, I, 61).to(gpu)
    enc.dn_q = torch.from_numpy(mo.preshuffle_ns_down(enc.dn_q.cpu().numpy())).to(gpu)
    enc.dn_ns = True
    dec = wl.make_experts(E, H, I, 61).to(gpu)
    for name in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z"):
        setattr(dec, name, getattr(enc, name))
    dec.dn_ns = True
    hidden = wl.make_hidden(T, H, 62).to(gpu)
    ids, w = wl.make_routing(T, E, tk, 63)
    ids, w = ids.to(gpu), w.to(gpu)
    y0 = v2.fused_moe_w4_v2(hidden, plain, ids, w)
    y1 = v2.fused_moe_w4_v2(hidden, enc, ids, w)
    y2 = v2.fused_moe_w4_v2(hidden, dec, ids, w)
    torch.cuda.synchronize()
    assert enc.dn_q is dec.dn_q and enc.dn_tiled and dec.dn_tiled
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert torch.equal(y0.view(torch.int16), y2.view(torch.int16))


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


# ------------------------------------------------------------------ W4 quantisation and loading
def _edge_weights(N, K, gs, seed, dtype):
    """Random rows plus groups that exercise the corners of the rule: a
    constant group (range 0, scale from the 1e-8 floor), an all-positive group
    (zero clamps at 0), a group whose minimum is exactly 0 (zero = -0.0), an
    all-negative group (zero clamps at 15), large and tiny magnitudes."""
    g = torch.Generator().manual_seed(seed)
    W = 0.02 * torch.randn(N, K, generator=g)
    W[0, :gs] = 0.37
    W[1, :gs] = torch.rand(gs, generator=g) + 0.5
    W[2, :gs] = torch.rand(gs, generator=g)
    W[2, 3] = 0.0
    W[3, :gs] = -torch.rand(gs, generator=g) - 0.5
    W[4, :gs] = 1e3 * torch.randn(gs, generator=g)
    W[5, :gs] = 1e-6 * torch.randn(gs, generator=g)
    return W.to(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("E,N,K,gs", [(2, 64, 2816, 128), (3, 48, 704, 64), (1, 16, 256, 32)])
def test_quantize_w4_matches_the_oracle(gpu, dtype, E, N, K, gs):
    w4 = load_mod("w4a16")
    W = torch.stack([_edge_weights(N, K, gs, 50 + e, dtype) for e in range(E)])
    print(f"ksl_quantize_w4 {dtype} E={E} N={N} K={K} gs={gs}", flush=True)
    q, s, z = w4.quantize_w4(W.to(gpu), gs)
    torch.cuda.synchronize()
    rq, rs, rz = mo.quantize_w4(W.float().reshape(E * N, K).numpy(), gs)
    assert np.array_equal(q.cpu().numpy().reshape(E * N, K // 2), rq)
    assert np.array_equal(s.cpu().numpy().reshape(E * N, -1).view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(z.cpu().numpy().reshape(E * N, -1).view(np.uint16), rz.view(np.uint16))
    # the group whose minimum is 0 keeps the reference's -0.0 zero-point
    assert z.cpu()[0, 2, 0].view(torch.int16).item() == -32768


class _Experts(torch.nn.Module):
    """A bf16 experts module as the model holds it before packing."""

    def __init__(self, E, H, I, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.gate_up_proj = torch.nn.Parameter((0.02 * torch.randn(E, 2 * I, H, generator=g)).to(torch.bfloat16),
                                               requires_grad=False)
        self.down_proj = torch.nn.Parameter((0.02 * torch.randn(E, H, I, generator=g)).to(torch.bfloat16),
                                            requires_grad=False)
        self.act_fn = torch.nn.functional.silu


def test_pack_experts_module_quantises_as_the_reference(gpu):
    pe = load_mod("pack_experts")
    wl = load_mod("workloads")
    E, H, I, T, tk = 8, 256, 192, 24, 4
    exp = _Experts(E, H, I, 60).to(gpu)
    gu_ref = mo.quantize_w4(exp.gate_up_proj.float().cpu().numpy().reshape(E * 2 * I, H), 128)
    dn_ref = mo.quantize_w4(exp.down_proj.float().cpu().numpy().reshape(E * H, I), 64)
    pe.pack_experts_module(exp)
    assert exp.gate_up_proj is None and exp.down_proj is None and exp.dn_tiled
    assert np.array_equal(exp.gu_q.cpu().numpy().reshape(E * 2 * I, -1), gu_ref[0])
    assert np.array_equal(exp.gu_s.cpu().numpy().reshape(E * 2 * I, -1).view(np.uint16), gu_ref[1].view(np.uint16))
    assert np.array_equal(exp.gu_z.cpu().numpy().reshape(E * 2 * I, -1).view(np.uint16), gu_ref[2].view(np.uint16))
    dn_q = mo.untile_down(exp.dn_q.cpu().numpy(), I)
    assert np.array_equal(dn_q.reshape(E * H, -1), dn_ref[0])
    assert np.array_equal(exp.dn_z.cpu().numpy().reshape(E * H, -1).view(np.uint16), dn_ref[2].view(np.uint16))
    hidden = wl.make_hidden(T, H, 61).to(gpu)
    ids, w = wl.make_routing(T, E, tk, 62)
    y = exp(hidden, ids.to(gpu), w.to(gpu))  # the bound fused forward
    torch.cuda.synchronize()
    assert y.shape == (T, H) and bool(torch.isfinite(y.float()).all())


class _Layer(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.experts = torch.nn.Module()
        self.experts.act_fn = torch.nn.functional.silu


class _Model(torch.nn.Module):
    """Encoder and decoder stacks whose layer N experts share one shard."""

    def __init__(self, L):
        super().__init__()
        self.encoder = torch.nn.Module()
        self.decoder = torch.nn.Module()
        self.encoder.layers = torch.nn.ModuleList([_Layer() for _ in range(L)])
        self.decoder.layers = torch.nn.ModuleList([_Layer() for _ in range(L)])


def test_bind_expert_shards_shares_one_tensor_per_layer(gpu, tmp_path):
    from safetensors.torch import save_file
    lw = load_mod("load_w4")
    v2 = load_mod("fused_moe_w4_v2")
    wl = load_mod("workloads")
    L, E, H, I, T, tk = 2, 8, 256, 192, 16, 4
    plain = []
    for i in range(L):
        exp = wl.make_experts(E, H, I, 70 + i)
        plain.append(exp.to(gpu))
        prefix = f"model.decoder.layers.{i}.experts"
        save_file({f"{prefix}.{b}": getattr(exp, b).contiguous() for b in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z")},
                  str(tmp_path / f"experts_{i:03d}.safetensors"))
    model = _Model(L).to(gpu)
    (tmp_path / "w4_meta.json").write_text('{"format": "dg-w4a16-v1"}')
    assert lw.bind_expert_shards(model, tmp_path, device=gpu, pack=True) == 2 * L
    hidden = wl.make_hidden(T, H, 72).to(gpu)
    ids, w = wl.make_routing(T, E, tk, 73)
    ids, w = ids.to(gpu), w.to(gpu)
    for i in range(L):
        enc, dec = model.encoder.layers[i].experts, model.decoder.layers[i].experts
        for b in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z", "gu_pack", "dn_pack"):
            assert getattr(enc, b).data_ptr() == getattr(dec, b).data_ptr(), b
        assert enc.dn_tiled and dec.dn_tiled
        y_enc = enc(hidden, ids, w)
        y_dec = dec(hidden, ids, w)
        y_ref = v2.fused_moe_w4_v2(hidden, plain[i], ids, w)
        torch.cuda.synchronize()
        assert torch.equal(y_enc.view(torch.int16), y_ref.view(torch.int16))
        assert torch.equal(y_dec.view(torch.int16), y_ref.view(torch.int16))
