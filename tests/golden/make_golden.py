"""Writes the golden fixtures of this directory from the oracle (the reference
ships no golden vectors for this path; its kill-tests are seeded-random with
tolerance gates). Inputs are seeded and small; every array is stored as plain
numeric data (np.savez_compressed, loaded with allow_pickle=False).

  rmsnorm_small.npz : x bf16 bits [16, 640], w bf16 bits [640], eps, y bf16
                      bits with w and without w (kernels/fused_rmsnorm.py:10-32)
  align_small.npz   : topk_ids int64 [10, 3] (two dropped ids), E = 5, and the
                      moe_align outputs for block_m 1 and 4
                      (kernels/fused_moe_w4.py:15-51)
  layer_small.npz   : RMSNorm + W4A16 MoE layer, T = 10, topk = 2, E = 4,
                      H = 256, I = 192, SiLU and tanh-GELU: packed experts,
                      routing, and y (fp32 combine, bf16 bits) per activation

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import moe_oracle as mo  # noqa: E402


def _bf16(x: np.ndarray) -> np.ndarray:
    return mo.f32_to_bf16(x.astype(np.float32))


def rmsnorm_small(rng):
    x = _bf16(2 * rng.standard_normal((16, 640)))
    w = _bf16(1 + 0.1 * rng.standard_normal(640))
    eps = np.float32(1e-6)
    y_w = mo.rmsnorm(mo.bf16_to_f32(x), mo.bf16_to_f32(w), float(eps))
    y_nw = mo.rmsnorm(mo.bf16_to_f32(x), None, float(eps))
    return dict(x=x, w=w, eps=eps, y_w=y_w, y_nw=y_nw)


def align_small(rng):
    ids = rng.integers(0, 5, size=(10, 3)).astype(np.int64)
    ids[2, 1] = 5
    ids[7, 0] = 9
    out = dict(ids=ids, E=np.int64(5))
    for bm in (1, 4):
        sr, eids, cap, inv = mo.moe_align(ids, bm, 5)
        out.update({f"sorted_rows_bm{bm}": sr, f"expert_ids_bm{bm}": eids, f"cap_bm{bm}": np.int64(cap),
                    f"inv_bm{bm}": inv})
    return out


def layer_small(rng):
    T, tk, E, H, I = 10, 2, 4, 256, 192
    x = _bf16(rng.standard_normal((T, H)))
    norm_w = _bf16(1 + 0.1 * rng.standard_normal(H))
    gu_q = rng.integers(0, 256, size=(E, 2 * I, H // 2), dtype=np.uint8)
    gu_s = rng.uniform(0.005, 0.02, size=(E, 2 * I, H // 128)).astype(np.float16)
    gu_z = rng.integers(0, 16, size=(E, 2 * I, H // 128)).astype(np.float16)
    dn_q = rng.integers(0, 256, size=(E, H, I // 2), dtype=np.uint8)
    dn_s = rng.uniform(0.005, 0.02, size=(E, H, I // 64)).astype(np.float16)
    dn_z = rng.integers(0, 16, size=(E, H, I // 64)).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:tk] for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.1, 1.0, size=(T, tk)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    xn = mo.rmsnorm(mo.bf16_to_f32(x), mo.bf16_to_f32(norm_w), 1e-6)
    out = dict(x=x, norm_w=norm_w, eps=np.float32(1e-6), gu_q=gu_q, gu_s=gu_s, gu_z=gu_z, dn_q=dn_q, dn_s=dn_s,
               dn_z=dn_z, topk_ids=ids, topk_w=w, xn=xn)
    for name, act in (("silu", mo.ACT_SILU), ("gelu", mo.ACT_GELU_TANH)):
        y = mo.moe_forward(mo.bf16_to_f32(xn), gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, ids, w, act)
        out[f"y_{name}"] = y
        out[f"y_{name}_bf16"] = mo.f32_to_bf16(y)
    return out


def main():
    rng = np.random.default_rng(20261201)
    for name, fn in (("rmsnorm_small", rmsnorm_small), ("align_small", align_small), ("layer_small", layer_small)):
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **fn(rng))
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
