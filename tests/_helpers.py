"""Shared test utilities: bf16 bit access, ulp distances, normalised errors."""
from __future__ import annotations

import numpy as np
import torch


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    assert t.dtype == torch.bfloat16
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f16_bits(t: torch.Tensor) -> np.ndarray:
    assert t.dtype == torch.float16
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def bits_to_bf16_tensor(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def ordered16(b: np.ndarray) -> np.ndarray:
    """Map 16-bit float bit patterns to integers whose difference is the ulp distance."""
    b = b.astype(np.int64)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def ulp_diff16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.abs(ordered16(a) - ordered16(b))


def norm_err(out: np.ndarray, ref: np.ndarray):
    """(normalised max error, normalised mean error) — the reference's convention
    (kernels/pack_experts.py:152-156, kernels/fused_moe_w4_v2.py:393-394)."""
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = np.abs(out - ref)
    return float(d.max() / (np.abs(ref).max() + 1e-9)), float(d.mean() / (np.abs(ref).mean() + 1e-9))


# tolerances for the bf16/fp16 MoE outputs (normalised, reference convention)
MOE_MAX_TOL = 2e-2
MOE_MEAN_TOL = 1e-2


def act_unperm(a: np.ndarray, gs: int) -> np.ndarray:
    """Undo the expert-GEMM activation storage order along the last axis: within
    each group of gs elements, logical offset o = c*(gs/4) + i*8 + j is stored
    at i*32 + c*8 + s(j), with s the inverse of the K-slot order {0,4,1,5,2,6,3,7}."""
    n = a.shape[-1]
    q = gs // 4
    o = np.arange(n) % gs
    g0 = np.arange(n) - o
    c, i, j = o // q, (o % q) // 8, o % 8
    sj = np.where(j < 4, 2 * j, 2 * (j - 4) + 1)
    store = g0 + i * 32 + c * 8 + sj
    return a[..., store]


def out2_unperm(a: np.ndarray, I: int) -> np.ndarray:
    """Undo the out2 storage order: 128-element groups over the first I - I % 128
    columns, a 64-element group over the rest."""
    i128 = I - I % 128
    if i128 == I:
        return act_unperm(a, 128)
    return np.concatenate([act_unperm(a[..., :i128], 128), act_unperm(a[..., i128:], 64)], axis=-1)
