"""GPU routing metadata — drop-in for moe_align in kernels/fused_moe_w4.py.

  moe_align(topk_ids, block_m, E) -> (sorted_rows, expert_ids, cap, inv)
                                                     (kernels/fused_moe_w4.py:15-51)

Same outputs, bit for bit, built by one HIP launch instead of ~14 torch ops:
sorted_rows int64[cap] (expanded row t*topk+slot per sorted slot, pad =
T*topk), expert_ids int64[max_blocks] (pad = E), cap (python int, fixed from
the shapes, no sync), inv int64[T*topk] (sorted slot per expanded row,
dropped rows 0). Ids are clamped to <= E (E = dropped); the reference raises on
a negative id, this path treats it as dropped.

  fused_moe_w4(hidden, exp, topk_ids, topk_w) -> Tensor   (kernels/fused_moe_w4.py:104-128)

The reference's v1 forward, for experts whose activation is any callable
(exp.act_fn, applied between the two GEMMs as the reference does, :119):
routing and the fp16 activation copy (ksl_moe_route), the grouped gate/up GEMM
writing gate and up themselves (ksl_moe_gateup_act with KSL_ACT_NONE),
exp.act_fn(gate) * up in torch on the GPU (the caller's function), the rows
put into the down kernel's activation order (ksl_moe_act_to_down_order), the
grouped down GEMM (ksl_moe_down) and the v1 combine in fp16 products
(ksl_moe_combine_v1). The rows are kept compact per expert (no block_m
padding): each output row depends only on its own token, so the layout does
not change the values.
"""
from __future__ import annotations

import torch

from . import _lib

BLOCK_M = 64  # kernels/fused_moe_w4.py:12 (the v1 tile; v2 uses its own)


@torch.no_grad()
def moe_align(topk_ids: torch.Tensor, block_m: int, E: int):
    if topk_ids.dim() != 2:
        raise ValueError("topk_ids must be [T, topk]")
    T, tk = topk_ids.shape
    block_m = int(block_m)
    E = int(E)
    if block_m <= 0 or E <= 0:
        raise ValueError("block_m and E must be positive")
    if E > 512:
        raise ValueError("E > 512 experts is not supported")
    dev = topk_ids.device
    ids = topk_ids.to(torch.int64).contiguous()
    Nexp = T * tk
    max_blocks = (Nexp + block_m - 1) // block_m + E
    cap = max_blocks * block_m
    sorted_rows = torch.empty(cap, dtype=torch.int64, device=dev)
    expert_ids = torch.empty(max_blocks, dtype=torch.int64, device=dev)
    inv = torch.empty(Nexp, dtype=torch.int64, device=dev)
    rc = _lib.load().ksl_moe_align(_lib.ptr(ids), T, tk, E, block_m, _lib.ptr(sorted_rows),
                                   _lib.ptr(expert_ids), _lib.ptr(inv), _lib.stream_of(ids))
    _lib.check(rc, "ksl_moe_align")
    return sorted_rows, expert_ids, cap, inv


@torch.no_grad()
def fused_moe_w4(hidden: torch.Tensor, exp, topk_ids: torch.Tensor, topk_w: torch.Tensor) -> torch.Tensor:
    """kernels/fused_moe_w4.py:104-128: one MoE layer with the activation
    exp.act_fn applied in torch between the gate/up and down GEMMs. `exp`
    carries gu_q/gu_s/gu_z, dn_q/dn_s/dn_z in the packed format
    (kernels/pack_experts.py:96-97) and act_fn."""
    return expert_rows_forward(hidden, exp, topk_ids, topk_w, combine="v1")


@torch.no_grad()
def expert_rows_forward(hidden: torch.Tensor, exp, topk_ids: torch.Tensor, topk_w: torch.Tensor,
                        combine: str = "v1") -> torch.Tensor:
    """Routing, gate/up, exp.act_fn(gate) * up in torch, down, then the
    combine: "v1" the v1 fp16-product combine (kernels/fused_moe_w4.py:125-127,
    ksl_moe_combine_v1), "stock" the stock experts loop's expert-ordered
    index_add_ (kernels/pack_experts.py:44-62, ksl_moe_combine_stock)."""
    from .fused_moe_w4_v2 import _check_weights, _same_device, check_zero_points_once, dn_layout
    if combine not in ("v1", "stock"):
        raise ValueError(f"unknown combine {combine!r}")
    T, H = hidden.shape
    tk = topk_ids.shape[1]
    E, twoI, _ = exp.gu_q.shape
    I = twoI // 2
    Nexp = T * tk
    if not hidden.is_cuda:
        raise ValueError("hidden must be on the GPU")
    _check_weights(exp, E, H, I)
    check_zero_points_once(exp)
    _same_device(hidden.device, topk_ids=topk_ids, topk_w=topk_w, gu_q=exp.gu_q, dn_q=exp.dn_q)
    _lib.dtype_code(hidden.dtype), _lib.dtype_code(topk_w.dtype)  # fp32 / fp16 / bf16, else TypeError
    dev = hidden.device
    y = torch.empty(T, H, dtype=hidden.dtype, device=dev)
    if T == 0:
        return y
    lib = _lib.load()
    st = _lib.stream_of(hidden)
    ids = topk_ids.to(torch.int64).contiguous()
    w = topk_w.contiguous()
    aligned = hidden.stride(1) == 1 and hidden.stride(0) % 8 == 0 and hidden.data_ptr() % 16 == 0
    # a fresh allocation (16-byte aligned) where the routing launch cannot read in place
    x = hidden if aligned else torch.empty(T, H, dtype=hidden.dtype, device=dev).copy_(hidden)
    sorted_rows = torch.empty(Nexp, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    inv = torch.empty(Nexp, dtype=torch.int32, device=dev)
    a16 = torch.empty(T, H, dtype=torch.float16, device=dev)
    _lib.check(lib.ksl_moe_route(_lib.ptr(ids), T, tk, E, _lib.ptr(sorted_rows), _lib.ptr(offsets),
                                 _lib.ptr(inv), _lib.ptr(x), _lib.dtype_code(x.dtype), x.stride(0), H,
                                 _lib.ptr(a16), st), "ksl_moe_route")
    out1 = torch.empty(Nexp, twoI, dtype=torch.float16, device=dev)
    _lib.check(lib.ksl_moe_gateup_act(_lib.ptr(a16), _lib.ptr(sorted_rows), _lib.ptr(offsets), T, tk,
                                      _lib.ptr(exp.gu_q), _lib.ptr(exp.gu_s), _lib.ptr(exp.gu_z), E, H, I,
                                      _lib.ACT_NONE, _lib.ptr(out1), st), "ksl_moe_gateup_act")
    gate, up = out1.chunk(2, dim=-1)
    out2 = (exp.act_fn(gate) * up).to(torch.float16).contiguous()  # :119, [Nexp, I]
    out2d = torch.empty_like(out2)
    _lib.check(lib.ksl_moe_act_to_down_order(_lib.ptr(out2), Nexp, I, _lib.ptr(out2d), st),
               "ksl_moe_act_to_down_order")
    out3 = torch.empty(Nexp, H, dtype=torch.float16, device=dev)
    _lib.check(lib.ksl_moe_down(_lib.ptr(out2d), _lib.ptr(offsets), _lib.ptr(exp.dn_q), _lib.ptr(exp.dn_s),
                                _lib.ptr(exp.dn_z), E, H, I, Nexp, _lib.ptr(out3), dn_layout(exp), st),
               "ksl_moe_down")
    if combine == "v1":
        _lib.check(lib.ksl_moe_combine_v1(_lib.ptr(out3), _lib.ptr(inv), _lib.ptr(w), _lib.dtype_code(w.dtype), T,
                                          tk, H, _lib.ptr(y), _lib.dtype_code(y.dtype), H, st), "ksl_moe_combine_v1")
    else:
        _lib.check(lib.ksl_moe_combine_stock(_lib.ptr(out3), _lib.ptr(inv), _lib.ptr(ids), E, _lib.ptr(w),
                                             _lib.dtype_code(w.dtype), T, tk, H, _lib.ptr(y),
                                             _lib.dtype_code(y.dtype), H, st), "ksl_moe_combine_stock")
    return y
