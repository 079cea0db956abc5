"""GPU parity for the expert router (the step before the MoE), through the C ABI
and the drop-in router_forward.

Bars: probabilities within 1e-2 relative everywhere and within 1e-5 for >= 99%
of them (a score may round to the neighbouring bf16 value when the GPU's fp32
accumulation order differs from the oracle's exact sum: about 0.4% on that
probability); top-k equal to the oracle's up to ties and near-ties at the k-th
value (1e-2 relative), with equal weights for the ids both pick; bit-identical
reruns.
"""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from tests._helpers import assert_topk_equivalent
from tests.conftest import load_mod, load_pkg

pytestmark = pytest.mark.gpu


def _params(E, H, seed):
    g = torch.Generator().manual_seed(seed)
    scale = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    proj = (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16)
    pes = (1 + 0.1 * torch.randn(E, generator=g)).to(torch.bfloat16)
    return scale, proj, pes


def _run(x, scale, proj, pes, k, eps=1e-6):
    lib = load_pkg()._lib
    L = lib.load()
    T, H = x.shape
    E = proj.shape[0]
    probs = torch.empty(T, E, dtype=torch.float32, device=x.device)
    w = torch.empty(T, k, dtype=torch.float32, device=x.device)
    ids = torch.empty(T, k, dtype=torch.int64, device=x.device)
    rc = L.ksl_moe_router(lib.ptr(x), lib.dtype_code(x.dtype), x.stride(0), lib.ptr(scale), lib.ptr(proj),
                          lib.ptr(pes), lib.DTYPE_BF16, eps, T, H, E, k, lib.ptr(probs), lib.ptr(w), lib.ptr(ids),
                          lib.stream_of(x))
    lib.check(rc, "ksl_moe_router")
    torch.cuda.synchronize()
    return probs, w, ids


CASES = [
    # (T, H, E, k, seed, x dtype)
    (256, 2816, 128, 8, 41, torch.bfloat16),   # the 256-token canvas
    (1, 2816, 128, 8, 42, torch.bfloat16),
    (37, 512, 32, 4, 43, torch.bfloat16),      # ragged token count (rows past T in the last workgroup)
    (200, 256, 64, 2, 44, torch.float16),
    (20, 4096, 256, 16, 45, torch.bfloat16),   # largest supported sizes
    (64, 1056, 128, 8, 48, torch.bfloat16),    # 33 K steps: only the first projection wave has a 5th
    (16, 2848, 64, 6, 49, torch.bfloat16),     # 89 K steps, 6 column steps with a partial last one
    (9, 32, 16, 2, 50, torch.float16),         # smallest row (one K step) and one expert tile
]


@pytest.mark.parametrize("T,H,E,k,seed,xd", CASES)
def test_router_vs_oracle(gpu, T, H, E, k, seed, xd):
    print(f"router T={T} H={H} E={E} k={k} {xd}", flush=True)
    scale, proj, pes = _params(E, H, seed)
    x = (2 * torch.randn(T, H, generator=torch.Generator().manual_seed(seed + 1))).to(xd)
    probs, w, ids = _run(x.to(gpu), scale.to(gpu), proj.to(gpu), pes.to(gpu), k)
    po, wo, io = mo.router(x.float().numpy(), scale.float().numpy(), proj.float().numpy(), pes.float().numpy(),
                           1e-6, k)
    p = probs.cpu().numpy()
    rel = np.abs(p - po) / po
    print(f"  probs rel max {rel.max():.2e}, frac > 1e-5: {(rel > 1e-5).mean():.4f}; ids equal rows "
          f"{(ids.cpu().numpy() == io).all(-1).mean():.3f}")
    assert rel.max() <= 1e-2 and (rel > 1e-5).mean() <= 0.01
    assert_topk_equivalent(po, io, wo, ids.cpu().numpy(), w.cpu().numpy(), rtol=1e-2, boundary_rtol=1e-2)
    probs2, w2, ids2 = _run(x.to(gpu), scale.to(gpu), proj.to(gpu), pes.to(gpu), k)
    assert torch.equal(probs, probs2) and torch.equal(w, w2) and torch.equal(ids, ids2)


def test_router_ties_take_lower_ids(gpu):
    """Zero projection: every probability 1/E; the picks are ids 0..k-1 with
    weight per_expert_scale / k (the oracle's tie rule)."""
    T, H, E, k = 40, 512, 64, 8
    scale, _, pes = _params(E, H, 46)
    proj = torch.zeros(E, H, dtype=torch.bfloat16)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(47)).to(torch.bfloat16)
    probs, w, ids = _run(x.to(gpu), scale.to(gpu), proj.to(gpu), pes.to(gpu), k)
    assert torch.all(probs.cpu() == 1.0 / E)
    assert torch.equal(ids.cpu(), torch.arange(k).expand(T, k))
    ref = pes.float()[:k] / k
    assert torch.allclose(w.cpu(), ref.expand(T, k), rtol=1e-6)


def test_router_drop_in_matches_stock_module(gpu):
    """router_forward bound on a stock DiffusionGemmaTextRouter (patch_routers)
    against the unpatched module run by torch on the GPU."""
    from transformers.models.diffusion_gemma.configuration_diffusion_gemma import DiffusionGemmaTextConfig
    from transformers.models.diffusion_gemma.modeling_diffusion_gemma import DiffusionGemmaTextRouter
    router = load_mod("router")
    E, H, k, T = 128, 2816, 8, 256
    cfg = DiffusionGemmaTextConfig(num_experts=E, hidden_size=H, top_k_experts=k, rms_norm_eps=1e-6)
    stock = DiffusionGemmaTextRouter(cfg).to(torch.bfloat16)
    scale, proj, pes = _params(E, H, 48)
    with torch.no_grad():
        stock.proj.weight.copy_(proj)
        stock.scale.copy_(scale)
        stock.per_expert_scale.copy_(pes)
    stock = stock.to(gpu)
    x = (2 * torch.randn(T, H, generator=torch.Generator().manual_seed(49))).to(torch.bfloat16).to(gpu)
    with torch.no_grad():
        p_ref, w_ref, i_ref = stock(x)
    holder = torch.nn.ModuleList([stock])
    assert router.patch_routers(holder, verbose=False) == 1
    p, w, i = stock(x)
    assert p.dtype == torch.float32 and w.dtype == torch.float32 and i.dtype == torch.int64
    assert p.shape == (T, E) and w.shape == (T, k) and i.shape == (T, k)
    rel = (p - p_ref).abs() / p_ref
    print(f"drop-in: probs rel max {rel.max().item():.2e}; ids equal rows "
          f"{(i == i_ref).all(-1).float().mean().item():.3f}")
    assert rel.max().item() <= 2e-2
    assert_topk_equivalent(p_ref.cpu().numpy(), i_ref.cpu().numpy(), w_ref.cpu().numpy(), i.cpu().numpy(),
                           w.cpu().numpy(), rtol=2e-2, boundary_rtol=2e-2)
