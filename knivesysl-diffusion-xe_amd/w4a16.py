"""Load-time W4 quantisation — drop-in for quantize_w4 and dequant_w4 in kernels/w4a16.py.

  quantize_w4(W, group_size=128) -> (qpacked uint8, scale fp16, zero fp16)
                                                    (kernels/w4a16.py:19-32)
  dequant_w4(qpacked, scale, zero, group_size=128) -> W fp16
                                                    (kernels/w4a16.py:35-48)

Runs ksl_quantize_w4 on the GPU: asymmetric 4-bit per (row, group of
group_size columns along K), the same bytes, scales and zero-points as the
reference. W may be [N, K] or an expert stack [E, N, K] (each expert's rows
quantised as the reference's _pack_3d does one expert at a time,
kernels/pack_experts.py:34-41; rows are independent, so the stack is one
launch). bf16, fp16 and fp32 weights are read as they are (converted to fp32
exactly inside the kernel).
"""
from __future__ import annotations

import torch

from . import _lib

GS = 128


@torch.no_grad()
def quantize_w4(W: torch.Tensor, group_size: int = GS):
    """W [..., N, K] on the GPU -> (qpacked uint8 [..., N, K/2], scale fp16
    [..., N, K/gs], zero fp16 [..., N, K/gs])."""
    if not W.is_cuda:
        raise ValueError("quantize_w4 runs on the GPU: move W to a cuda device")
    if W.dim() < 2:
        raise ValueError("W must be [N, K] or [E, N, K]")
    K = W.shape[-1]
    if K % group_size != 0:
        raise ValueError(f"K = {K} is not a multiple of group_size = {group_size}")
    lead = tuple(W.shape[:-1])
    Wc = W.contiguous()
    rows = Wc.numel() // K
    q = torch.empty(lead + (K // 2,), dtype=torch.uint8, device=W.device)
    s = torch.empty(lead + (K // group_size,), dtype=torch.float16, device=W.device)
    z = torch.empty_like(s)
    rc = _lib.load().ksl_quantize_w4(_lib.ptr(Wc), _lib.dtype_code(Wc.dtype), rows, K, group_size, _lib.ptr(q),
                                     _lib.ptr(s), _lib.ptr(z), _lib.stream_of(Wc))
    _lib.check(rc, "ksl_quantize_w4")
    return q, s, z


@torch.no_grad()
def dequant_w4(qpacked: torch.Tensor, scale: torch.Tensor, zero: torch.Tensor, group_size: int = GS):
    """qpacked uint8 [..., N, K/2], scale / zero fp16 [..., N, K/gs] on the GPU
    -> W fp16 [..., N, K] = fp16((q - zero) * scale), bit for bit the
    reference's torch expression (ksl_dequant_w4)."""
    if not qpacked.is_cuda:
        raise ValueError("dequant_w4 runs on the GPU: move the buffers to a cuda device")
    if qpacked.dtype != torch.uint8 or scale.dtype != torch.float16 or zero.dtype != torch.float16:
        raise TypeError("qpacked must be uint8, scale and zero float16")
    K = qpacked.shape[-1] * 2
    if K % group_size != 0:
        raise ValueError(f"K = {K} is not a multiple of group_size = {group_size}")
    lead = tuple(qpacked.shape[:-1])
    if tuple(scale.shape) != lead + (K // group_size,) or tuple(zero.shape) != tuple(scale.shape):
        raise ValueError(f"scale / zero must be {lead + (K // group_size,)}")
    q, sc, zr = qpacked.contiguous(), scale.contiguous(), zero.contiguous()
    out = torch.empty(lead + (K,), dtype=torch.float16, device=qpacked.device)
    rows = q.numel() // (K // 2) if K else 0
    rc = _lib.load().ksl_dequant_w4(_lib.ptr(q), _lib.ptr(sc), _lib.ptr(zr), rows, K, group_size, _lib.ptr(out),
                                    _lib.stream_of(q))
    _lib.check(rc, "ksl_dequant_w4")
    return out
