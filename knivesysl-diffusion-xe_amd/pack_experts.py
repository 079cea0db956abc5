"""Experts forward binding — drop-in for fused_experts_forward in kernels/pack_experts.py.

  fused_experts_forward(self, hidden_states, top_k_index, top_k_weights)
                                                   (kernels/pack_experts.py:65-84)
is bound per DiffusionGemmaTextExperts module by the loader
(kernels/load_w4_checkpoint.py:83) and always runs the fused HIP forward (the
reference's MOE_V2=1 branch, :80-82; its v1 fallback is superseded).
GU_GS / DN_GS are the pack's group sizes (kernels/pack_experts.py:12).
"""
from __future__ import annotations

from .fused_moe_w4_v2 import fused_moe_w4_v2

GU_GS, DN_GS = 128, 64


def fused_experts_forward(self, hidden_states, top_k_index, top_k_weights):
    return fused_moe_w4_v2(hidden_states, self, top_k_index, top_k_weights)
