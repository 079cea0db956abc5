"""Host logic of the drop-in modules, on the CPU: activation selection and the
reference's error behaviour; nothing here falls back to a CPU computation."""
from __future__ import annotations

import pytest
import torch

from tests.conftest import load_mod


class _Exp:
    def __init__(self, act_fn):
        self.act_fn = act_fn


@pytest.mark.parametrize("name,code", [("gelu_pytorch_tanh", 0), ("gelu_new", 0), ("gelu", 0), ("silu", 1)])
def test_activation_selection(name, code):
    from transformers.activations import ACT2FN
    v2 = load_mod("fused_moe_w4_v2")
    e = _Exp(ACT2FN[name])
    assert v2._check_act(e) and e._ksl_act == code and e._act_checked


def test_unsupported_activation_raises():
    from transformers.activations import ACT2FN
    v2 = load_mod("fused_moe_w4_v2")
    with pytest.raises(AssertionError, match="tanh-GELU and SiLU"):
        v2._check_act(_Exp(ACT2FN["relu"]))


def test_shape_asserts_like_the_reference():
    v2 = load_mod("fused_moe_w4_v2")
    wl = load_mod("workloads")
    exp = wl.make_experts(2, 256, 128, 0)
    ids = torch.zeros(4, 2, dtype=torch.int64)
    w = torch.ones(4, 2)
    with pytest.raises(AssertionError, match="divisible by 128"):
        v2.fused_moe_w4_v2(torch.zeros(4, 200, dtype=torch.bfloat16), exp, ids, w)
    exp_bad_i = wl.make_experts(2, 256, 96, 0)
    with pytest.raises(AssertionError, match="divisible by 64"):
        v2.fused_moe_w4_v2(torch.zeros(4, 256, dtype=torch.bfloat16), exp_bad_i, ids, w)


def test_cpu_tensors_fail_loudly():
    v2 = load_mod("fused_moe_w4_v2")
    fr = load_mod("fused_rmsnorm")
    wl = load_mod("workloads")
    exp = wl.make_experts(2, 256, 128, 0)
    with pytest.raises(ValueError, match="GPU"):
        v2.fused_moe_w4_v2(torch.zeros(4, 256, dtype=torch.bfloat16), exp, torch.zeros(4, 2, dtype=torch.int64),
                           torch.ones(4, 2))
    with pytest.raises((ValueError, RuntimeError)):
        fr.fused_rmsnorm(torch.zeros(4, 256, dtype=torch.bfloat16), None, 1e-6)


def test_patch_rmsnorms_binds_the_fused_forward():
    from transformers.models.diffusion_gemma.modeling_diffusion_gemma import DiffusionGemmaRMSNorm
    fr = load_mod("fused_rmsnorm")
    model = torch.nn.Sequential(DiffusionGemmaRMSNorm(64), torch.nn.Linear(64, 64),
                                DiffusionGemmaRMSNorm(64, with_scale=False))
    n = fr.patch_rmsnorms(model, verbose=False)
    assert n == 2
    for m in (model[0], model[2]):
        assert m.forward.__func__ is fr._fused_forward


def test_workload_shapes():
    wl = load_mod("workloads")
    exp = wl.make_experts(4, 256, 128, 1)
    assert tuple(exp.gu_q.shape) == (4, 256, 128) and exp.gu_q.dtype == torch.uint8
    assert tuple(exp.gu_s.shape) == (4, 256, 2) and exp.gu_s.dtype == torch.float16
    assert tuple(exp.dn_q.shape) == (4, 256, 64) and tuple(exp.dn_s.shape) == (4, 256, 2)
    z = torch.cat([exp.gu_z.flatten(), exp.dn_z.flatten()])
    assert bool(((z == z.round()) & (z >= 0) & (z <= 15)).all())
    ids, w = wl.make_routing(16, 4, 2, 2)
    assert ids.shape == (16, 2) and ids.dtype == torch.int64
    assert torch.allclose(w.sum(-1), torch.ones(16))
    a, b = wl.make_routing(16, 4, 2, 2)
    assert torch.equal(a, ids) and torch.equal(b, w)  # seeded


def test_moe_block_forward_checks_dtypes_and_patches_layers():
    mb = load_mod("moe_block")
    with pytest.raises(TypeError, match="bf16"):
        mb.moe_block_forward(None, torch.zeros(4, 256), torch.zeros(4, 256))
    with pytest.raises(ValueError, match="shapes"):
        mb.moe_block_forward(None, torch.zeros(4, 256, dtype=torch.bfloat16), torch.zeros(4, 128, dtype=torch.bfloat16))

    # only layers whose experts carry the packed buffers are rebound
    class DiffusionGemmaDecoderTextLayer(torch.nn.Module):
        def __init__(self, packed):
            super().__init__()
            self.experts = torch.nn.Module()
            if packed:
                self.experts.gu_q = torch.zeros(1, dtype=torch.uint8)

    model = torch.nn.ModuleList([DiffusionGemmaDecoderTextLayer(True), DiffusionGemmaDecoderTextLayer(False)])
    assert mb.patch_moe_blocks(model, verbose=False) == 1
    assert model[0].forward.__func__ is mb.layer_forward
    assert "forward" not in model[1].__dict__


def test_checkpoint_meta_refuses_a_directory_without_w4_meta(tmp_path):
    """kernels/load_w4_checkpoint.py:38-41: a directory without w4_meta.json
    is not a dg-w4a16 checkpoint (checked before anything is loaded)."""
    lw = load_mod("load_w4")
    with pytest.raises(AssertionError, match="not a dg-w4a16 checkpoint"):
        lw.checkpoint_meta(tmp_path)
    with pytest.raises(AssertionError, match="not a dg-w4a16 checkpoint"):
        lw.bind_expert_shards(torch.nn.Module(), tmp_path, device="cpu")
    (tmp_path / "w4_meta.json").write_text('{"format": "dg-w4a16-v1", "group_size": 128}')
    assert lw.checkpoint_meta(tmp_path)["format"] == "dg-w4a16-v1"
    (tmp_path / "w4_meta.json").write_text('[1, 2]')
    with pytest.raises(ValueError):
        lw.checkpoint_meta(tmp_path)
