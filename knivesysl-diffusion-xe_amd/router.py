"""Expert router on the GPU (the step before the MoE): drop-in for the stock
DiffusionGemmaTextRouter.forward (TF modeling_diffusion_gemma.py:529-548).

The reference leaves the router to stock torch (about eight launches: its
norm, two scalings, the projection, softmax, top-k, the renormalisation and the
per-expert scale); here one launch of libksl.so computes the same outputs, with
the router's scale-free norm as the fused RMSNorm (the reference patches every
DiffusionGemmaRMSNorm, kernels/load_w4_checkpoint.py:126-127).
"""
from __future__ import annotations

import torch

from . import _lib


@torch.no_grad()
def router_forward(self, hidden_states: torch.Tensor):
    """(router_probabilities fp32 [T, E], top_k_weights fp32 [T, k],
    top_k_index int64 [T, k]) as DiffusionGemmaTextRouter.forward returns them."""
    x = hidden_states.reshape(-1, hidden_states.shape[-1])
    if x.stride(-1) != 1 or x.stride(0) % 8 != 0 or x.data_ptr() % 16 != 0:
        x = x.clone(memory_format=torch.contiguous_format)  # a fresh, aligned copy
    T, H = x.shape
    proj = self.proj.weight
    E = proj.shape[0]
    k = int(self.config.top_k_experts)
    params = []
    for t in (self.scale, proj, self.per_expert_scale):
        if t.dtype != torch.bfloat16 or t.device != x.device:
            raise TypeError("router parameters must be bf16 tensors on the hidden states' device")
        params.append(t.contiguous())
    scale, proj, pes = params
    probs = torch.empty(T, E, dtype=torch.float32, device=x.device)
    topk_w = torch.empty(T, k, dtype=torch.float32, device=x.device)
    topk_ids = torch.empty(T, k, dtype=torch.int64, device=x.device)
    rc = _lib.load().ksl_moe_router(_lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), _lib.ptr(scale),
                                    _lib.ptr(proj), _lib.ptr(pes), _lib.DTYPE_BF16, float(self.eps), T, H, E, k,
                                    _lib.ptr(probs), _lib.ptr(topk_w), _lib.ptr(topk_ids), _lib.stream_of(x))
    _lib.check(rc, "ksl_moe_router")
    return probs, topk_w, topk_ids


def patch_routers(model, verbose: bool = True) -> int:
    """Rebind forward of every DiffusionGemmaTextRouter in `model` to
    router_forward (the way patch_rmsnorms rebinds the norms). Returns the count."""
    n = 0
    for mod in model.modules():
        if type(mod).__name__ == "DiffusionGemmaTextRouter":
            mod.forward = router_forward.__get__(mod, mod.__class__)
            n += 1
    if verbose:
        print(f"[router] patched {n} routers")
    return n
