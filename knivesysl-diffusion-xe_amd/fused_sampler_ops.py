"""Per-step sampler kernels on gfx950 — drop-in for kernels/fused_sampler_ops.py.

  fused_entropy(logits) -> entropy               (kernels/fused_sampler_ops.py:43-51)
  gumbel_argmax_sample(logits, seed) -> (sampled, argmax)   (:84-93)
  sample_step(logits, seed) -> (sampled, argmax, entropy)   (both, one read of the logits)

logits [..., V] fp32 (or bf16 / fp16) on the GPU. The sample is the
Gumbel-max draw with Triton's tl.rand(seed + row, column) noise, restated
exactly (Philox4x32-10), so a given seed gives the reference's draws; the
argmax is exact (first index of the max). Entropy is fp32, nats; entries
equal to -inf contribute nothing (as torch's Categorical.entropy; the
reference's kernel returns NaN for such rows). One C call per function, no
host sync.
"""
from __future__ import annotations

import torch

from . import _lib


def _rows(logits: torch.Tensor) -> torch.Tensor:
    x = logits.reshape(-1, logits.shape[-1])
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


@torch.no_grad()
def fused_entropy(logits: torch.Tensor) -> torch.Tensor:
    """logits [..., V] -> entropy [...] fp32 (nats), one pass."""
    x = _rows(logits)
    rows, V = x.shape
    h = torch.empty(rows, dtype=torch.float32, device=x.device)
    rc = _lib.load().ksl_entropy(_lib.ptr(x), _lib.dtype_code(x.dtype), rows, V, x.stride(0) if rows else V,
                                 _lib.ptr(h), _lib.stream_of(x))
    _lib.check(rc, "ksl_entropy")
    return h.view(logits.shape[:-1])


@torch.no_grad()
def gumbel_argmax_sample(logits: torch.Tensor, seed: int):
    """logits [..., V] -> (sampled idx, argmax idx) int64 [...]. Gumbel-max ==
    Categorical sample; seed is an integer (the row's generator key is seed + row)."""
    x = _rows(logits)
    rows, V = x.shape
    samp = torch.empty(rows, dtype=torch.int64, device=x.device)
    amax = torch.empty(rows, dtype=torch.int64, device=x.device)
    rc = _lib.load().ksl_gumbel_argmax(_lib.ptr(x), _lib.dtype_code(x.dtype), rows, V,
                                       x.stride(0) if rows else V, int(seed), _lib.ptr(samp), _lib.ptr(amax),
                                       _lib.stream_of(x))
    _lib.check(rc, "ksl_gumbel_argmax")
    return samp.view(logits.shape[:-1]), amax.view(logits.shape[:-1])


@torch.no_grad()
def sample_step(logits: torch.Tensor, seed: int):
    """gumbel_argmax_sample and fused_entropy from one read of the logits:
    (sampled, argmax, entropy)."""
    x = _rows(logits)
    rows, V = x.shape
    samp = torch.empty(rows, dtype=torch.int64, device=x.device)
    amax = torch.empty(rows, dtype=torch.int64, device=x.device)
    h = torch.empty(rows, dtype=torch.float32, device=x.device)
    rc = _lib.load().ksl_sample_step(_lib.ptr(x), _lib.dtype_code(x.dtype), rows, V, x.stride(0) if rows else V,
                                     int(seed), _lib.ptr(samp), _lib.ptr(amax), _lib.ptr(h), _lib.stream_of(x))
    _lib.check(rc, "ksl_sample_step")
    shape = logits.shape[:-1]
    return samp.view(shape), amax.view(shape), h.view(shape)
