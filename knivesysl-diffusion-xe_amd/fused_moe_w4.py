"""GPU routing metadata — drop-in for moe_align in kernels/fused_moe_w4.py.

  moe_align(topk_ids, block_m, E) -> (sorted_rows, expert_ids, cap, inv)
                                                     (kernels/fused_moe_w4.py:15-51)

Same outputs, bit for bit, built by one HIP launch instead of ~14 torch ops:
sorted_rows int64[cap] (expanded row t*topk+slot per sorted slot, pad =
T*topk), expert_ids int64[max_blocks] (pad = E), cap (python int, fixed from
the shapes, no sync), inv int64[T*topk] (sorted slot per expanded row,
dropped rows 0). Ids are clamped to <= E (E = dropped); the reference raises on
a negative id, this path treats it as dropped.

The v1 grouped kernel of the reference (fused_moe_w4 / _grouped_w4) is
superseded by fused_moe_w4_v2 and is not provided.
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
