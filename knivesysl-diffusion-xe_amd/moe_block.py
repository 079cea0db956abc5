"""The decoder layer's MoE branch and its tail on the GPU (the step after the MoE).

TF modeling_diffusion_gemma.py:729-743 (DiffusionGemmaDecoderTextLayer.forward;
the encoder layer's :651-665 is the same) runs, after the MLP branch:

    x  = residual                                   (hidden_states_flat)
    topk_w, topk_ids = router(x)
    m  = experts(pre_feedforward_layernorm_2(x), topk_ids, topk_w)
    y  = (residual + post_feedforward_layernorm(hidden_states_1
                      + post_feedforward_layernorm_2(m))) * layer_scalar

With the reference's bindings (kernels/load_w4_checkpoint.py:83, :126-127)
that is the router, one fused_rmsnorm, the fused MoE (four kernels), two more
fused_rmsnorm calls, two adds and the in-place scalar multiply. Here the
router is whatever `layer.router` is bound to, and one C call
(ksl_moe_block_forward) runs the rest in four launches: the tail is the
combine kernel's epilogue. Values: every element as the stock tail on the
fused RMSNorm, up to the row sums' fp32 order.
"""
from __future__ import annotations

import torch

from . import _lib
from .fused_moe_w4_v2 import _check_act, _check_weights, dn_layout, moe_workspace, pack_ptrs


def _rows(t: torch.Tensor, H: int) -> torch.Tensor:
    x = t.reshape(-1, H)
    if x.stride(-1) != 1 or x.stride(0) % 8 != 0 or x.data_ptr() % 16 != 0:
        x = x.clone(memory_format=torch.contiguous_format)  # a fresh, aligned copy
    return x


def _norm_weight(mod, name: str, dev, H: int) -> torch.Tensor:
    w = getattr(mod, "weight", None) if getattr(mod, "with_scale", True) else None
    if w is None:
        raise ValueError(f"{name}: a scaled RMSNorm is required")
    if w.dtype != torch.bfloat16 or w.device != dev or tuple(w.shape) != (H,):
        raise TypeError(f"{name}.weight must be bf16 [{H}] on {dev}")
    return w.contiguous()


@torch.no_grad()
def moe_block_forward(layer, residual: torch.Tensor, hidden_states_1: torch.Tensor) -> torch.Tensor:
    """The layer output of TF modeling_diffusion_gemma.py:729-743 for one
    DiffusionGemma{Decoder,Encoder}TextLayer, given its residual stream
    (`residual`, bf16 [..., H]) and the MLP branch's normalised output
    (`hidden_states_1`, same shape). `layer.experts` holds the reference's
    packed W4 buffers (gu_q, gu_s, gu_z, dn_q, dn_s, dn_z). Returns a new bf16
    tensor of residual's shape."""
    if residual.dtype != torch.bfloat16 or hidden_states_1.dtype != torch.bfloat16:
        raise TypeError("moe_block_forward: residual and hidden_states_1 must be bf16")
    if hidden_states_1.shape != residual.shape:
        raise ValueError("moe_block_forward: hidden_states_1 and residual shapes differ")
    H = residual.shape[-1]
    dev = residual.device
    x = _rows(residual, H)
    h1 = _rows(hidden_states_1, H)
    T = x.shape[0]
    _, topk_w, topk_ids = layer.router(x)
    exp = layer.experts
    E, twoI, _ = exp.gu_q.shape
    I = twoI // 2
    if H % 128 != 0 or I % 64 != 0:
        raise ValueError(f"hidden {H} must be divisible by 128 and expert intermediate {I} by 64")
    if not getattr(exp, "_act_checked", False) or not hasattr(exp, "_ksl_act"):
        _check_act(exp)
    _check_weights(exp, E, H, I)
    pre = layer.pre_feedforward_layernorm_2
    post2 = layer.post_feedforward_layernorm_2
    post = layer.post_feedforward_layernorm
    pre_w = _norm_weight(pre, "pre_feedforward_layernorm_2", dev, H)
    post2_w = _norm_weight(post2, "post_feedforward_layernorm_2", dev, H)
    post_w = _norm_weight(post, "post_feedforward_layernorm", dev, H)
    ls = getattr(layer, "layer_scalar", None)
    if ls is not None:
        if ls.numel() != 1 or ls.device != dev or ls.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError("layer_scalar must be one fp32 or bf16 element on the hidden states' device")
        ls = ls.contiguous()
    ids = topk_ids if topk_ids.dtype == torch.int64 else topk_ids.to(torch.int64)
    ids = ids.contiguous()
    w = topk_w.contiguous()
    tk = ids.shape[1]
    y = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    if T == 0:
        return y.reshape(residual.shape)
    ws = moe_workspace(T, tk, E, H, I, dev)
    rc = _lib.load().ksl_moe_block_forward(
        _lib.ptr(x), x.stride(0), _lib.ptr(pre_w), float(pre.eps),
        _lib.ptr(ids), _lib.ptr(w), _lib.dtype_code(w.dtype),
        _lib.ptr(exp.gu_q), _lib.ptr(exp.gu_s), _lib.ptr(exp.gu_z),
        _lib.ptr(exp.dn_q), _lib.ptr(exp.dn_s), _lib.ptr(exp.dn_z), dn_layout(exp), *pack_ptrs(exp),
        T, tk, E, H, I, exp._ksl_act,
        _lib.ptr(h1), h1.stride(0), _lib.ptr(post2_w), float(post2.eps), _lib.ptr(post_w), float(post.eps),
        _lib.ptr(ls), _lib.DTYPE_BF16 if ls is None else _lib.dtype_code(ls.dtype),
        _lib.ptr(y), y.stride(0), _lib.ptr(ws), ws.numel(), _lib.stream_of(x))
    _lib.check(rc, "ksl_moe_block_forward")
    return y.reshape(residual.shape)


def layer_forward(self, hidden_states: torch.Tensor, position_embeddings: torch.Tensor = None,
                  attention_mask: torch.Tensor | None = None, position_ids: torch.LongTensor | None = None,
                  past_key_values=None, **kwargs) -> torch.Tensor:
    """DiffusionGemma{Decoder,Encoder}TextLayer.forward (TF
    modeling_diffusion_gemma.py:700-744, :621-666): attention and the MLP
    branch through the layer's own modules, then moe_block_forward."""
    residual = hidden_states
    hidden_states = self.input_layernorm(hidden_states)
    hidden_states, _ = self.self_attn(hidden_states=hidden_states, position_embeddings=position_embeddings,
                                      attention_mask=attention_mask, position_ids=position_ids,
                                      past_key_values=past_key_values, **kwargs)
    hidden_states = self.post_attention_layernorm(hidden_states)
    hidden_states = residual + hidden_states
    residual = hidden_states
    hidden_states = self.pre_feedforward_layernorm(hidden_states)
    hidden_states = self.mlp(hidden_states)
    hidden_states_1 = self.post_feedforward_layernorm_1(hidden_states)
    return moe_block_forward(self, residual, hidden_states_1)


_LAYER_CLASSES = ("DiffusionGemmaDecoderTextLayer", "DiffusionGemmaEncoderTextLayer")


def patch_moe_blocks(model, verbose: bool = True) -> int:
    """Rebind forward of every DiffusionGemma decoder/encoder text layer whose
    experts hold the packed W4 buffers to layer_forward (as patch_rmsnorms
    rebinds the norms, kernels/fused_rmsnorm.py:39-48). Returns the count."""
    n = 0
    for mod in model.modules():
        if type(mod).__name__ in _LAYER_CLASSES and hasattr(getattr(mod, "experts", None), "gu_q"):
            mod.forward = layer_forward.__get__(mod, mod.__class__)
            n += 1
    if verbose:
        print(f"[moe-block] patched {n} layers")
    return n
