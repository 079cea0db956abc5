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

pack_experts_module / pack_all_experts (kernels/pack_experts.py:87-122)
quantise a bf16 experts module in place with the GPU quantiser
(w4a16.quantize_w4): the six packed buffers, the tiled down layout, the
fused forward bound.
"""
from __future__ import annotations

import torch

from .fused_moe_w4_v2 import enable_tiled_down, fused_moe_w4_v2
from .w4a16 import quantize_w4

GU_GS, DN_GS = 128, 64
EXPERT_BUFS = ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z")  # kernels/load_w4_checkpoint.py:27


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


@torch.no_grad()
def pack_experts_module(exp, free_bf16: bool = True, cache: dict | None = None):
    """Quantise one experts module in place (kernels/pack_experts.py:87-106):
    gate_up_proj [E, 2I, H] in groups of GU_GS along H, down_proj [E, H, I] in
    groups of DN_GS along I, as the six buffers the fused forward reads; the
    down weights then go to the tiled layout (enable_tiled_down, which also
    checks the zero-points), and the fused forward is bound. free_bf16 drops
    the bf16 weights."""
    gu = quantize_w4(exp.gate_up_proj.data, GU_GS)
    dn = quantize_w4(exp.down_proj.data, DN_GS)
    for name, t in zip(EXPERT_BUFS, gu + dn):
        exp.register_buffer(name, t, persistent=False)
    if free_bf16:
        exp.gate_up_proj = None
        exp.down_proj = None
    enable_tiled_down(exp, cache)
    exp.forward = fused_experts_forward.__get__(exp, exp.__class__)
    return exp


@torch.no_grad()
def pack_all_experts(model, free_bf16: bool = True, verbose: bool = True) -> int:
    """pack_experts_module on every module with bf16 expert weights
    (gate_up_proj and down_proj, kernels/pack_experts.py:109-122)."""
    n, gu_elems, dn_elems = 0, 0, 0
    for mod in model.modules():
        gp, dp = getattr(mod, "gate_up_proj", None), getattr(mod, "down_proj", None)
        if isinstance(gp, torch.Tensor) and isinstance(dp, torch.Tensor) and gp.dim() == 3:
            gu_elems += gp.numel()
            dn_elems += dp.numel()
            pack_experts_module(mod, free_bf16)
            n += 1
    if verbose:
        gib = 2 ** 30
        print(f"[pack] {n} experts modules -> W4 (gate/up gs{GU_GS}, down gs{DN_GS}): "
              f"{2 * (gu_elems + dn_elems) / gib:.2f} GiB bf16 -> {(gu_elems + dn_elems) / 2 / gib:.2f} GiB W4",
              flush=True)
    return n
