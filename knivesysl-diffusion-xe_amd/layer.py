"""RMSNorm + W4A16 MoE layer: the measured hot path.

In a DiffusionGemma MoE layer the experts consume
pre_feedforward_layernorm_2(residual) (TF modeling_diffusion_gemma.py:731-733):
  x_n = fused_rmsnorm(x, norm_w, eps)                     (kernels/fused_rmsnorm.py:24)
  y   = fused_moe_w4_v2(x_n, exp, topk_ids, topk_w)       (kernels/fused_moe_w4_v2.py:320)
Five launches on the current stream (norm, route+prep, gate/up, down,
combine), no host sync.

LayerRunner issues the same five launches one C call at a time, with a
preallocated workspace, so a caller can record HIP events between them.
"""
from __future__ import annotations

import torch

from . import _lib
from .fused_moe_w4_v2 import _check_act, _check_weights, fused_moe_w4_v2
from .fused_rmsnorm import fused_rmsnorm

STAGES = ("rmsnorm", "route", "gateup", "down", "combine")


@torch.no_grad()
def moe_layer(x: torch.Tensor, norm_w: torch.Tensor | None, eps: float, exp, topk_ids: torch.Tensor,
              topk_w: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    xn = fused_rmsnorm(x, norm_w, eps)
    return fused_moe_w4_v2(xn, exp, topk_ids, topk_w, workspace=workspace)


class LayerRunner:
    """Preallocated buffers for one (T, topk, E, H, I) layer shape."""

    def __init__(self, T: int, topk: int, E: int, H: int, I: int, device, act_dtype=torch.bfloat16):
        self.T, self.topk, self.E, self.H, self.I = T, topk, E, H, I
        self.device = torch.device(device)
        nexp = T * topk
        self.xn = torch.empty(T, H, dtype=act_dtype, device=device)
        self.sorted_rows = torch.empty(nexp, dtype=torch.int32, device=device)
        self.offsets = torch.empty(E + 1, dtype=torch.int32, device=device)
        self.inv = torch.empty(nexp, dtype=torch.int32, device=device)
        self.a16 = torch.empty(T, H, dtype=torch.float16, device=device)
        self.out2 = torch.empty(nexp, I, dtype=torch.float16, device=device)
        self.out3 = torch.empty(nexp, H, dtype=torch.float16, device=device)
        self.y = torch.empty(T, H, dtype=act_dtype, device=device)
        self.lib = _lib.load()

    @torch.no_grad()
    def run(self, x, norm_w, eps, exp, topk_ids, topk_w, events=None):
        """events: optional list of 6 torch.cuda.Event recorded before, between
        and after the five launches."""
        L, p = self.lib, _lib.ptr
        T, tk, E, H, I = self.T, self.topk, self.E, self.H, self.I
        if not getattr(exp, "_act_checked", False) or not hasattr(exp, "_ksl_act"):
            _check_act(exp)
        _check_weights(exp, E, H, I)
        st = _lib.stream_of(x)
        code = _lib.dtype_code(x.dtype)
        ev = events
        if ev:
            ev[0].record()
        rc = L.ksl_rmsnorm(p(x), code, p(norm_w), _lib.dtype_code(norm_w.dtype) if norm_w is not None else code,
                           p(self.xn), code, T, H, x.stride(0), H, float(eps), st)
        _lib.check(rc, "ksl_rmsnorm")
        if ev:
            ev[1].record()
        rc = L.ksl_moe_route(p(topk_ids), T, tk, E, p(self.sorted_rows), p(self.offsets), p(self.inv),
                             p(self.xn), code, H, H, p(self.a16), st)
        _lib.check(rc, "ksl_moe_route")
        if ev:
            ev[2].record()
        rc = L.ksl_moe_gateup_act(p(self.a16), p(self.sorted_rows), p(self.offsets), tk, p(exp.gu_q),
                                  p(exp.gu_s), p(exp.gu_z), E, H, I, exp._ksl_act, p(self.out2), st)
        _lib.check(rc, "ksl_moe_gateup_act")
        if ev:
            ev[3].record()
        rc = L.ksl_moe_down(p(self.out2), p(self.offsets), p(exp.dn_q), p(exp.dn_s), p(exp.dn_z), E, H, I,
                            p(self.out3), st)
        _lib.check(rc, "ksl_moe_down")
        if ev:
            ev[4].record()
        rc = L.ksl_moe_combine(p(self.out3), p(self.inv), p(topk_w), _lib.dtype_code(topk_w.dtype), T, tk, H,
                               p(self.y), code, H, st)
        _lib.check(rc, "ksl_moe_combine")
        if ev:
            ev[5].record()
        return self.y
