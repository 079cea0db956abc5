"""The HIP path against the committed oracle fixtures (tests/golden)."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from tests._helpers import bits_to_bf16_tensor, bf16_bits, check_norm_err, ulp_diff16
from tests.conftest import load_mod

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
pytestmark = pytest.mark.gpu


def _load(name):
    return np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False)


def test_rmsnorm_vs_fixture(gpu):
    fr = load_mod("fused_rmsnorm")
    f = _load("rmsnorm_small")
    x = bits_to_bf16_tensor(f["x"]).to(gpu)
    w = bits_to_bf16_tensor(f["w"]).to(gpu)
    for wt, key in ((w, "y_w"), (None, "y_nw")):
        y = fr.fused_rmsnorm(x, wt, float(f["eps"]))
        d = ulp_diff16(bf16_bits(y.cpu()), f[key])
        assert d.max() <= 1 and (d == 0).mean() > 0.999


@pytest.mark.parametrize("bm", [1, 4])
def test_align_vs_fixture(gpu, bm):
    fm = load_mod("fused_moe_w4")
    f = _load("align_small")
    sr, eids, cap, inv = fm.moe_align(torch.from_numpy(f["ids"]).to(gpu), bm, int(f["E"]))
    assert cap == int(f[f"cap_bm{bm}"])
    assert np.array_equal(sr.cpu().numpy(), f[f"sorted_rows_bm{bm}"])
    assert np.array_equal(eids.cpu().numpy(), f[f"expert_ids_bm{bm}"])
    assert np.array_equal(inv.cpu().numpy(), f[f"inv_bm{bm}"])


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_layer_vs_fixture(gpu, act):
    layer = load_mod("layer")
    wl = load_mod("workloads")
    f = _load("layer_small")
    fn = wl.silu if act == "silu" else wl.gelu_pytorch_tanh
    exp = wl.Experts(*(torch.from_numpy(f[k]) for k in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z")),
                     act_fn=fn).to(gpu)
    x = bits_to_bf16_tensor(f["x"]).to(gpu)
    nw = bits_to_bf16_tensor(f["norm_w"]).to(gpu)
    ids = torch.from_numpy(f["topk_ids"]).to(gpu)
    w = torch.from_numpy(f["topk_w"]).to(gpu)
    y = layer.moe_layer(x, nw, float(f["eps"]), exp, ids, w)
    got = y.float().cpu().numpy()
    check_norm_err("layer_fixture", got, f[f"y_{act}"], act)
