"""GPU parity: HIP RMSNorm vs the oracle (kernels/fused_rmsnorm.py:10-32 semantics).

Bar: every output within 1 bf16 ulp of the oracle (the fp32 sum order differs),
>= 99% bit-exact; the bit-exact fraction is printed.
"""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as mo
from tests._helpers import bf16_bits, ulp_diff16
from tests.conftest import load_mod

pytestmark = pytest.mark.gpu


def _check(x_cpu, w_cpu, eps, gpu, min_exact=0.99):
    frm = load_mod("fused_rmsnorm")
    y = frm.fused_rmsnorm(x_cpu.to(gpu), None if w_cpu is None else w_cpu.to(gpu), eps)
    torch.cuda.synchronize()
    assert y.dtype == x_cpu.dtype and y.shape == x_cpu.shape
    x32 = x_cpu.float().numpy().reshape(-1, x_cpu.shape[-1])
    w32 = None if w_cpu is None else w_cpu.float().numpy()
    ref = mo.rmsnorm(x32, w32, eps)
    got = y.reshape(-1, x_cpu.shape[-1]).cpu()
    if got.dtype != torch.bfloat16:
        # non-bf16 x: value was rounded to bf16 then cast exactly
        got = got.to(torch.bfloat16)
    gb = bf16_bits(got)
    d = ulp_diff16(gb, ref)
    exact = float((d == 0).mean())
    print(f"rmsnorm {tuple(x_cpu.shape)} w={'yes' if w_cpu is not None else 'no'}: "
          f"max ulp {int(d.max())}, bit-exact {exact:.6f}")
    assert d.max() <= 1
    assert exact >= min_exact
    return exact


def test_rmsnorm_256_canvas(gpu):
    wl = load_mod("workloads")
    x, w, eps = wl.rmsnorm_256(0)
    _check(x, w, eps, gpu)


def test_rmsnorm_32k_outliers_and_qk(gpu):
    wl = load_mod("workloads")
    x, w, qk, qk_w, eps = wl.rmsnorm_32k(1)
    _check(x, w, eps, gpu)
    _check(qk, qk_w, eps, gpu)


def test_rmsnorm_no_scale_and_shapes(gpu):
    g = torch.Generator().manual_seed(5)
    x = (0.3 * torch.randn(1, 256, 16, 256, generator=g)).to(torch.bfloat16)
    _check(x, None, 1e-6, gpu)
    w = (0.5 * torch.randn(256, generator=g)).to(torch.bfloat16)
    _check(x, w, 1e-6, gpu)
    x = torch.randn(1, 768, 2816, generator=g).to(torch.bfloat16)
    _check(x, (torch.randn(2816, generator=g) * 0.5).to(torch.bfloat16), 1e-6, gpu)


def test_rmsnorm_ragged_cols_scalar_path(gpu):
    g = torch.Generator().manual_seed(6)
    for cols in (1, 7, 100, 2817):
        x = torch.randn(33, cols, generator=g).to(torch.bfloat16)
        _check(x, (1 + 0.1 * torch.randn(cols, generator=g)).to(torch.bfloat16), 1e-6, gpu)


def test_rmsnorm_long_rows_two_pass(gpu):
    g = torch.Generator().manual_seed(7)
    x = torch.randn(9, 8192, generator=g).to(torch.bfloat16)
    _check(x, (1 + 0.1 * torch.randn(8192, generator=g)).to(torch.bfloat16), 1e-6, gpu)


def test_rmsnorm_dtypes(gpu):
    g = torch.Generator().manual_seed(8)
    x = torch.randn(64, 2816, generator=g)
    w = (1 + 0.1 * torch.randn(2816, generator=g))
    _check(x.to(torch.float16), w.to(torch.bfloat16), 1e-6, gpu)
    _check(x, w, 1e-6, gpu)  # fp32 x, fp32 w


def test_rmsnorm_empty_and_noncontiguous(gpu):
    frm = load_mod("fused_rmsnorm")
    x = torch.empty(0, 2816, dtype=torch.bfloat16, device=gpu)
    y = frm.fused_rmsnorm(x, None, 1e-6)
    assert y.shape == (0, 2816)
    g = torch.Generator().manual_seed(9)
    base = torch.randn(64, 2 * 2816, generator=g).to(torch.bfloat16)
    xs = base[:, :2816]  # strided view; wrapper makes it contiguous like the reference
    _check(xs.contiguous(), None, 1e-6, gpu)
    y2 = frm.fused_rmsnorm(xs.to(gpu), None, 1e-6)
    y3 = frm.fused_rmsnorm(xs.contiguous().to(gpu), None, 1e-6)
    assert torch.equal(y2, y3)


def test_rmsnorm_zero_row(gpu):
    frm = load_mod("fused_rmsnorm")
    x = torch.zeros(4, 2816, dtype=torch.bfloat16, device=gpu)
    y = frm.fused_rmsnorm(x, torch.ones(2816, dtype=torch.bfloat16, device=gpu), 1e-6)
    assert torch.count_nonzero(y).item() == 0


def test_rmsnorm_deterministic(gpu):
    wl = load_mod("workloads")
    frm = load_mod("fused_rmsnorm")
    x, w, eps = wl.rmsnorm_256(0)
    a = frm.fused_rmsnorm(x.to(gpu), w.to(gpu), eps)
    b = frm.fused_rmsnorm(x.to(gpu), w.to(gpu), eps)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert np.array_equal(bf16_bits(a.cpu()), bf16_bits(b.cpu()))
