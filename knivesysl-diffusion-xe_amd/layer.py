"""RMSNorm + W4A16 MoE layer: the measured hot path.

In a DiffusionGemma MoE layer the experts consume
pre_feedforward_layernorm_2(residual) (TF modeling_diffusion_gemma.py:731-733):
  x_n = fused_rmsnorm(x, norm_w, eps)                     (kernels/fused_rmsnorm.py:24)
  y   = fused_moe_w4_v2(x_n, exp, topk_ids, topk_w)       (kernels/fused_moe_w4_v2.py:320)

moe_layer runs both as one C call on the current stream, no host sync:
(1) routing + RMSNorm + fp16 activations, (2) the experts: gate/up +
activation and down as ONE persistent launch when the experts carry the pack
layout (enable_pack) and at most 8192 rows are routed, else gate/up and down
as two launches, (3) fixed-order combine. The values are those of the two
separate calls (the norm is rounded to bf16 before the fp16 conversion, as
fused_rmsnorm's output is), which moe_layer_unfused runs for comparison.

LayerRunner issues the same launches one C call at a time, with preallocated
buffers, so a caller can record HIP events between them.
"""
from __future__ import annotations

import torch

from . import _lib
from .fused_moe_w4_v2 import (_check_act, _check_weights, _same_device, check_zero_points_once, dn_layout,
                              fused_moe_w4_v2, moe_workspace, pack_ptrs)
from .fused_rmsnorm import fused_rmsnorm

STAGES = ("route_norm", "gateup", "down", "combine")
STAGES_FFN = ("route_norm", "ffn", "combine")
FFN_MAX_ROWS = 8192  # routed rows up to which the one-launch expert FFN runs


def _prepare(exp, x, E, H, I):
    if not getattr(exp, "_act_checked", False) or not hasattr(exp, "_ksl_act"):
        _check_act(exp)
    _check_weights(exp, E, H, I)
    check_zero_points_once(exp)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("moe_layer takes bf16 or fp16 activations")
    if x.stride(1) != 1 or x.stride(0) % 8 != 0 or x.data_ptr() % 16 != 0:
        x = x.clone(memory_format=torch.contiguous_format)  # a fresh, aligned copy
    return x


@torch.no_grad()
def moe_layer(x: torch.Tensor, norm_w: torch.Tensor | None, eps: float, exp, topk_ids: torch.Tensor,
              topk_w: torch.Tensor, workspace: torch.Tensor | None = None) -> torch.Tensor:
    T, H = x.shape
    tk = topk_ids.shape[1]
    E, twoI, _ = exp.gu_q.shape
    I = twoI // 2
    x = _prepare(exp, x, E, H, I)
    if topk_ids.shape[0] != T or tuple(topk_w.shape) != tuple(topk_ids.shape):
        raise ValueError("topk_ids / topk_w must be [T, topk]")
    _same_device(x.device, topk_ids=topk_ids, topk_w=topk_w, norm_w=norm_w, gu_q=exp.gu_q)
    ids = topk_ids if topk_ids.dtype == torch.int64 else topk_ids.to(torch.int64)
    ids = ids.contiguous()
    w = topk_w.contiguous()
    nw = None if norm_w is None else norm_w.reshape(-1).contiguous()
    y = torch.empty(T, H, dtype=x.dtype, device=x.device)
    if T == 0:
        return y
    if workspace is None:
        workspace = moe_workspace(T, tk, E, H, I, x.device)
    rc = _lib.load().ksl_moe_layer_forward(
        _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), _lib.ptr(nw),
        _lib.dtype_code(nw.dtype) if nw is not None else _lib.DTYPE_BF16, float(eps),
        _lib.ptr(ids), _lib.ptr(w), _lib.dtype_code(w.dtype),
        _lib.ptr(exp.gu_q), _lib.ptr(exp.gu_s), _lib.ptr(exp.gu_z),
        _lib.ptr(exp.dn_q), _lib.ptr(exp.dn_s), _lib.ptr(exp.dn_z), dn_layout(exp), *pack_ptrs(exp),
        T, tk, E, H, I, exp._ksl_act, _lib.ptr(y), _lib.dtype_code(y.dtype), y.stride(0),
        _lib.ptr(workspace), workspace.numel(), _lib.stream_of(x))
    _lib.check(rc, "ksl_moe_layer_forward")
    return y


@torch.no_grad()
def moe_layer_unfused(x, norm_w, eps, exp, topk_ids, topk_w, workspace=None):
    """The same layer as two drop-in calls (norm, then the MoE forward)."""
    xn = fused_rmsnorm(x, norm_w, eps)
    return fused_moe_w4_v2(xn, exp, topk_ids, topk_w, workspace=workspace)


class LayerRunner:
    """Preallocated buffers for one (T, topk, E, H, I) layer shape. run()
    issues the launches of moe_layer one C call at a time: routing + RMSNorm,
    then either the one-launch expert FFN (experts with a pack, at most 8192
    routed rows: stages STAGES_FFN) or gate/up and down (STAGES), then the
    combine."""

    def __init__(self, T: int, topk: int, E: int, H: int, I: int, device, act_dtype=torch.bfloat16):
        self.T, self.topk, self.E, self.H, self.I = T, topk, E, H, I
        self.device = torch.device(device)
        self.act_dtype = act_dtype
        nexp = T * topk
        self.sorted_rows = torch.empty(nexp, dtype=torch.int32, device=device)
        self.offsets = torch.empty(E + 1, dtype=torch.int32, device=device)
        self.inv = torch.empty(nexp, dtype=torch.int32, device=device)
        self.a16 = torch.empty(T, H, dtype=torch.float16, device=device)
        self.out2 = torch.empty(nexp, I, dtype=torch.float16, device=device)
        self.out3 = torch.empty(nexp, H, dtype=torch.float16, device=device)
        self.y = torch.empty(T, H, dtype=act_dtype, device=device)
        self.lib = _lib.load()
        # block counts of the multi-block routing (above 4096 routed rows)
        self.scratch = torch.empty(max(1, int(self.lib.ksl_moe_route_scratch_bytes(T, topk, E)) // 4),
                                   dtype=torch.int32, device=device)
        # counters of the one-launch expert FFN: zero once, left zero by every launch
        self.ctl = torch.zeros(int(self.lib.ksl_moe_ffn_ctl_bytes(E)) // 4, dtype=torch.int32, device=device)

    def ffn_error(self) -> bool:
        """True if a one-launch FFN stage of this runner gave up a bounded wait
        (its out2 / out3 were then not to be trusted). The word latches until
        clear_ffn_error(); reading it synchronises with the device."""
        return bool(self.ctl[_lib.FFN_ERROR_WORD].item())

    def clear_ffn_error(self) -> None:
        self.ctl[_lib.FFN_ERROR_WORD] = 0

    def stages(self, exp) -> tuple:
        return STAGES_FFN if self._use_ffn(exp) else STAGES

    def _use_ffn(self, exp) -> bool:
        return (getattr(exp, "gu_pack", None) is not None and getattr(exp, "dn_pack", None) is not None
                and self.T * self.topk <= FFN_MAX_ROWS)

    @torch.no_grad()
    def run(self, x, norm_w, eps, exp, topk_ids, topk_w, events=None):
        """events: optional list of len(self.stages(exp)) + 1 torch.cuda.Event
        recorded before, between and after the launches."""
        L, p = self.lib, _lib.ptr
        T, tk, E, H, I = self.T, self.topk, self.E, self.H, self.I
        x = _prepare(exp, x, E, H, I)
        if x.dtype != self.act_dtype:
            raise TypeError(f"LayerRunner was built for {self.act_dtype} activations, got {x.dtype}")
        if tuple(topk_ids.shape) != (T, tk) or tuple(topk_w.shape) != (T, tk):
            raise ValueError(f"topk_ids / topk_w must be [{T}, {tk}]")
        if x.device != self.device:
            raise ValueError(f"x is on {x.device}, the runner's buffers on {self.device}")
        _same_device(x.device, topk_ids=topk_ids, topk_w=topk_w, norm_w=norm_w, gu_q=exp.gu_q)
        ids = topk_ids if topk_ids.dtype == torch.int64 else topk_ids.to(torch.int64)
        ids = ids.contiguous()
        w = topk_w.contiguous()
        nw = None if norm_w is None else norm_w.reshape(-1).contiguous()
        st = _lib.stream_of(x)
        code = _lib.dtype_code(x.dtype)
        ev = events
        k = 0
        if ev:
            ev[k].record()
        rc = L.ksl_moe_layer_route(p(ids), T, tk, E, p(self.sorted_rows), p(self.offsets), p(self.inv),
                                   p(x), code, x.stride(0), p(nw),
                                   _lib.dtype_code(nw.dtype) if nw is not None else code, float(eps),
                                   H, p(self.a16), p(self.scratch), self.scratch.numel() * 4, st)
        _lib.check(rc, "ksl_moe_layer_route")
        k += 1
        if ev:
            ev[k].record()
        if self._use_ffn(exp):
            rc = L.ksl_moe_ffn(p(self.a16), p(self.sorted_rows), p(self.offsets), T, tk, p(exp.gu_pack),
                               p(exp.dn_pack), E, H, I, exp._ksl_act, p(self.out2), p(self.out3), p(self.ctl), st)
            _lib.check(rc, "ksl_moe_ffn")
            k += 1
            if ev:
                ev[k].record()
        else:
            rc = L.ksl_moe_gateup_act(p(self.a16), p(self.sorted_rows), p(self.offsets), T, tk, p(exp.gu_q),
                                      p(exp.gu_s), p(exp.gu_z), E, H, I, exp._ksl_act, p(self.out2), st)
            _lib.check(rc, "ksl_moe_gateup_act")
            k += 1
            if ev:
                ev[k].record()
            rc = L.ksl_moe_down(p(self.out2), p(self.offsets), p(exp.dn_q), p(exp.dn_s), p(exp.dn_z), E, H, I,
                                T * tk, p(self.out3), dn_layout(exp), st)
            _lib.check(rc, "ksl_moe_down")
            k += 1
            if ev:
                ev[k].record()
        rc = L.ksl_moe_combine(p(self.out3), p(self.inv), p(w), _lib.dtype_code(w.dtype), T, tk, H,
                               p(self.y), code, H, st)
        _lib.check(rc, "ksl_moe_combine")
        k += 1
        if ev:
            ev[k].record()
        return self.y
