"""Experts forward binding — drop-in for fused_experts_forward in kernels/pack_experts.py.

  fused_experts_forward(self, hidden_states, top_k_index, top_k_weights)
                                                   (kernels/pack_experts.py:65-84)
is bound per DiffusionGemmaTextExperts module by the loader
(kernels/load_w4_checkpoint.py:83) and always runs the fused HIP forward (the
reference's MOE_V2=1 branch, :80-82; its v1 fallback is superseded).
GU_GS / DN_GS are the pack's group sizes (kernels/pack_experts.py:12).

repack_experts(model) is the load-time repack (after the loader binds the
packed buffers, kernels/load_w4_checkpoint.py:76-83): every experts module's
down weights go to the tiled layout the down kernel loads, once per buffer,
so the encoder and decoder modules that share a layer's tensors
(:56-59) keep sharing one repacked tensor.
"""
from __future__ import annotations

from .fused_moe_w4_v2 import enable_tiled_down, fused_moe_w4_v2

GU_GS, DN_GS = 128, 64


def fused_experts_forward(self, hidden_states, top_k_index, top_k_weights):
    return fused_moe_w4_v2(hidden_states, self, top_k_index, top_k_weights)


def repack_experts(model, verbose: bool = True) -> int:
    """Tile the down weights of every module holding the packed buffers
    (gu_q .. dn_z) in place; returns the number of modules. Idempotent."""
    cache: dict = {}
    n = 0
    for mod in model.modules():
        if hasattr(mod, "gu_q") and hasattr(mod, "dn_q"):
            enable_tiled_down(mod, cache)
            n += 1
    if verbose:
        print(f"[repack] {n} experts modules, {len(cache)} down buffers tiled")
    return n
