"""The committed fixtures (tests/golden/*.npz, written by make_golden.py from
the oracle) are reproduced bit for bit by the oracle and by the C restatement:
a regression pin on the oracle that the GPU parity tests compare against."""
from __future__ import annotations

import os

import numpy as np

from oracle import moe_oracle as mo
from oracle import oracle_c

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False)


def test_rmsnorm_fixture():
    f = _load("rmsnorm_small")
    x, w = mo.bf16_to_f32(f["x"]), mo.bf16_to_f32(f["w"])
    assert np.array_equal(mo.rmsnorm(x, w, float(f["eps"])), f["y_w"])
    assert np.array_equal(mo.rmsnorm(x, None, float(f["eps"])), f["y_nw"])


def test_align_fixture():
    f = _load("align_small")
    for bm in (1, 4):
        for impl in (mo.moe_align, oracle_c.moe_align):
            sr, eids, cap, inv = impl(f["ids"], bm, int(f["E"]))
            assert cap == int(f[f"cap_bm{bm}"])
            assert np.array_equal(sr, f[f"sorted_rows_bm{bm}"])
            assert np.array_equal(eids, f[f"expert_ids_bm{bm}"])
            assert np.array_equal(inv, f[f"inv_bm{bm}"])


def test_layer_fixture():
    f = _load("layer_small")
    xn = mo.rmsnorm(mo.bf16_to_f32(f["x"]), mo.bf16_to_f32(f["norm_w"]), float(f["eps"]))
    assert np.array_equal(xn, f["xn"])
    parts = [f[k] for k in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z")]
    for name, act in (("silu", mo.ACT_SILU), ("gelu", mo.ACT_GELU_TANH)):
        y = mo.moe_forward(mo.bf16_to_f32(xn), *parts, f["topk_ids"], f["topk_w"], act)
        assert np.array_equal(y, f[f"y_{name}"])
        assert np.array_equal(mo.f32_to_bf16(y), f[f"y_{name}_bf16"])
