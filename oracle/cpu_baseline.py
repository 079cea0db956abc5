"""The reference CPU path of the layer, in torch eager on the host cores.

TEST / MEASUREMENT INFRASTRUCTURE ONLY: timed by bench.py's cpu_baseline leg,
never called by the product.

Restated from:
- stock RMSNorm op sequence (TF modeling_diffusion_gemma.py:147-165): x.float(),
  pow(2).mean + eps, * pow(ms, -0.5), * w.float(), cast back;
- dequant_w4 (kernels/w4a16.py:35-48): W = fp16((q - z) * s);
- the per-expert loop of packed_experts_forward (kernels/pack_experts.py:44-62):
  gather the expert's rows, gate/up linear, act(gate) * up, down linear;
- the fixed top-k-slot-order combine (kernels/fused_moe_w4_v2.py:255-263).
The GEMMs run as fp32 MKL GEMMs on fp16-valued operands (fp16 GEMMs are not
native on the host CPU) with results rounded to fp16 where the reference
stores fp16.
"""
from __future__ import annotations

import os
import time

import torch
import torch.nn.functional as F


def host_threads() -> int:
    """Every core of this process's affinity set (the host's share for the run)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, n)


def rmsnorm_stock(x: torch.Tensor, w: torch.Tensor | None, eps: float) -> torch.Tensor:
    xf = x.float()
    ms = xf.pow(2).mean(-1, keepdim=True) + eps
    y = xf * torch.pow(ms, -0.5)
    if w is not None:
        y = y * w.float()
    return y.to(x.dtype)


def dequant_w4(q: torch.Tensor, s: torch.Tensor, z: torch.Tensor, gs: int) -> torch.Tensor:
    """fp16 weights [N, K] from the packed form, as fp32 tensor of fp16 values."""
    N, Kh = q.shape
    K = 2 * Kh
    codes = torch.empty(N, K, dtype=torch.float32)
    codes[:, 0::2] = (q & 0xF).float()
    codes[:, 1::2] = (q >> 4).float()
    W = (codes.view(N, K // gs, gs) - z.float()[..., None]) * s.float()[..., None]
    return W.view(N, K).half().float()


def _act(g: torch.Tensor, act: int) -> torch.Tensor:
    if act == 0:
        return 0.5 * g * (1.0 + torch.tanh(0.7978845608028654 * (g + 0.044715 * g * g * g)))
    return F.silu(g)


def moe_forward(hidden: torch.Tensor, exp, ids: torch.Tensor, w: torch.Tensor, act: int,
                predequant: list | None = None) -> torch.Tensor:
    """hidden [T,H] (bf16/fp16) -> [T,H] in hidden.dtype."""
    T, H = hidden.shape
    tk = ids.shape[1]
    E = exp.gu_q.shape[0]
    I = exp.gu_q.shape[1] // 2
    a = hidden.half().float()
    flat = ids.reshape(-1)
    out3 = torch.zeros(T * tk, H, dtype=torch.float32)
    for e in range(E):
        rows = torch.nonzero(flat == e).flatten()
        if rows.numel() == 0:
            continue
        if predequant is not None:
            wgu, wdn = predequant[e]
        else:
            wgu = dequant_w4(exp.gu_q[e], exp.gu_s[e], exp.gu_z[e], 128)
            wdn = dequant_w4(exp.dn_q[e], exp.dn_s[e], exp.dn_z[e], 64)
        x = a[rows // tk]
        gu = F.linear(x, wgu)
        h = (_act(gu[:, :I], act) * gu[:, I:]).half().float()
        out3[rows] = F.linear(h, wdn).half().float()
    acc = torch.zeros(T, H, dtype=torch.float32)
    out3 = out3.view(T, tk, H)
    wf = w.float()
    for k in range(tk):
        acc = acc + wf[:, k:k + 1] * out3[:, k]
    return acc.to(hidden.dtype)


def layer(x, norm_w, eps, exp, ids, w, act, predequant=None):
    return moe_forward(rmsnorm_stock(x, norm_w, eps), exp, ids, w, act, predequant)


def time_layer(x, norm_w, eps, exp, ids, w, act, budget_s: float = 20.0, max_runs: int = 5):
    """Median wall time (s) of the layer with dequant per call and with weights
    pre-dequantised, within about budget_s seconds. Returns a dict."""
    threads = host_threads()
    torch.set_num_threads(threads)
    res = {"threads": threads}
    t0 = time.perf_counter()
    with torch.no_grad():
        layer(x, norm_w, eps, exp, ids, w, act)  # warm-up
        runs = []
        while len(runs) < max_runs and (time.perf_counter() - t0) < budget_s * 0.6:
            s = time.perf_counter()
            layer(x, norm_w, eps, exp, ids, w, act)
            runs.append(time.perf_counter() - s)
        runs.sort()
        res["dequant_per_call_s"] = runs[len(runs) // 2]
        res["dequant_per_call_runs"] = len(runs)
        E = exp.gu_q.shape[0]
        pre = [(dequant_w4(exp.gu_q[e], exp.gu_s[e], exp.gu_z[e], 128),
                dequant_w4(exp.dn_q[e], exp.dn_s[e], exp.dn_z[e], 64)) for e in range(E)]
        layer(x, norm_w, eps, exp, ids, w, act, pre)
        runs = []
        t1 = time.perf_counter()
        while len(runs) < max_runs and (time.perf_counter() - t1) < budget_s * 0.3:
            s = time.perf_counter()
            layer(x, norm_w, eps, exp, ids, w, act, pre)
            runs.append(time.perf_counter() - s)
        runs.sort()
        res["predequant_s"] = runs[len(runs) // 2]
        res["predequant_runs"] = len(runs)
    res["wall_s"] = time.perf_counter() - t0
    return res
