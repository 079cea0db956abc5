"""Single-launch RMSNorm on gfx950 — drop-in for kernels/fused_rmsnorm.py.

Same names and call signatures as the reference module:
  fused_rmsnorm(x, weight, eps) -> Tensor          (kernels/fused_rmsnorm.py:24-32)
  _fused_forward(self, x)                           (kernels/fused_rmsnorm.py:35-36)
  patch_rmsnorms(model, verbose=True) -> int        (kernels/fused_rmsnorm.py:39-48)

Semantics: y = x / sqrt(mean(x^2) + eps) [* weight], fp32 accumulation, the
value rounded to bf16 and returned in x.dtype (the reference stores bf16 then
casts, :21 and :32). The HIP kernel writes x.dtype directly, one launch.
"""
from __future__ import annotations

import torch

from . import _lib


def fused_rmsnorm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    orig = x.shape
    x2 = x.reshape(-1, orig[-1]).contiguous()
    rows, n_cols = x2.shape
    y = torch.empty_like(x2)
    if weight is not None:
        if weight.device != x.device:
            raise ValueError("weight must be on the same device as x")
        w = weight.reshape(-1).contiguous()
        if w.numel() != n_cols:
            raise ValueError(f"weight has {w.numel()} elements, expected {n_cols}")
        wcode = _lib.dtype_code(w.dtype)
    else:
        w = None
        wcode = _lib.DTYPE_BF16
    xcode = _lib.dtype_code(x2.dtype)
    lib = _lib.load()
    rc = lib.ksl_rmsnorm(_lib.ptr(x2), xcode, _lib.ptr(w), wcode, _lib.ptr(y), xcode,
                         rows, n_cols, x2.stride(0) if rows else n_cols, y.stride(0) if rows else n_cols,
                         float(eps), _lib.stream_of(x2))
    _lib.check(rc, "ksl_rmsnorm")
    return y.reshape(orig)


def _fused_forward(self, x):
    return fused_rmsnorm(x, self.weight if self.with_scale else None, self.eps)


@torch.no_grad()
def patch_rmsnorms(model, verbose: bool = True) -> int:
    """Bind the fused forward on every DiffusionGemmaRMSNorm of `model`."""
    from transformers.models.diffusion_gemma.modeling_diffusion_gemma import DiffusionGemmaRMSNorm
    n = 0
    for mod in model.modules():
        if isinstance(mod, DiffusionGemmaRMSNorm):
            mod.forward = _fused_forward.__get__(mod, mod.__class__)
            n += 1
    if verbose:
        print(f"[fused-rmsnorm] patched {n} RMSNorm modules -> single HIP kernel", flush=True)
    return n
