"""Synthetic inputs of the benchmark workloads (seeded, generated with torch CPU
generators so that CPU and GPU see identical bits).

Shapes of the DiffusionGemma 26B-A4B MoE layer: H = 2816, I = 704, E = 128
experts, top-8, gate/up group 128, down group 64 (kernels/pack_experts.py:6, 12).

  rmsnorm_256     x bf16 [256, 2816] ~ N(0,1), w ~ N(1, 0.1), eps 1e-6
  rmsnorm_32k     x bf16 [32768, 2816] ~ N(0, 2), 0.1% of entries x50;
                  qk-norm x bf16 [4096, 256] ~ N(0,1) with its own w [256]
  gateup_256      A bf16 [256, 2816] ~ N(0,1); softmax(N(0,1) logits) top-8
                  renormalised; packed nibbles ~ U{0..15}; scale ~ U(0.005, 0.02);
                  zero ~ U{0..15}
  layer_256       RMSNorm (rmsnorm_256) then the full expert FFN + combine
  prefill_8192    T = 8192, logits biased so expert popularity follows
                  Zipf(s=1.1) over a seeded permutation of the 128 experts
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

H_DG, I_DG, E_DG, TOPK_DG = 2816, 704, 128, 8


def gelu_pytorch_tanh(x):
    return torch.nn.functional.gelu(x, approximate="tanh")


def silu(x):
    return torch.nn.functional.silu(x)


@dataclass
class Experts:
    """Duck-typed experts module with the packed W4 buffers (kernels/pack_experts.py:96-97)."""
    gu_q: torch.Tensor
    gu_s: torch.Tensor
    gu_z: torch.Tensor
    dn_q: torch.Tensor
    dn_s: torch.Tensor
    dn_z: torch.Tensor
    act_fn: object

    def to(self, device):
        return Experts(*(getattr(self, k).to(device) for k in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z")),
                       act_fn=self.act_fn)

    def nbytes(self) -> int:
        return sum(getattr(self, k).numel() * getattr(self, k).element_size()
                   for k in ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z"))


def _gen(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_experts(E: int, H: int, I: int, seed: int, act: str = "silu", device="cpu") -> Experts:
    """Random packed experts: every nibble ~ U{0..15} (a packed byte of two
    independent nibbles is U{0..255}), scale ~ U(0.005, 0.02) fp16,
    zero ~ U{0..15} fp16. Generated on `device` with a seeded generator."""
    g = _gen(seed, device)
    gu_q = torch.randint(0, 256, (E, 2 * I, H // 2), generator=g, dtype=torch.uint8, device=device)
    gu_s = (0.005 + 0.015 * torch.rand((E, 2 * I, H // 128), generator=g, device=device)).to(torch.float16)
    gu_z = torch.randint(0, 16, (E, 2 * I, H // 128), generator=g, device=device).to(torch.float16)
    dn_q = torch.randint(0, 256, (E, H, I // 2), generator=g, dtype=torch.uint8, device=device)
    dn_s = (0.005 + 0.015 * torch.rand((E, H, I // 64), generator=g, device=device)).to(torch.float16)
    dn_z = torch.randint(0, 16, (E, H, I // 64), generator=g, device=device).to(torch.float16)
    fn = silu if act == "silu" else gelu_pytorch_tanh
    return Experts(gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, fn)


def route(logits: torch.Tensor, k: int):
    """softmax(fp32) -> top-k -> renormalise (TF modeling_diffusion_gemma.py:538-547,
    per_expert_scale = 1). Returns (ids int64 [T,k], weights fp32 [T,k])."""
    p = torch.softmax(logits.float(), dim=-1, dtype=torch.float32)
    w, idx = torch.topk(p, k=k, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return idx.to(torch.int64), w


def make_routing(T: int, E: int, k: int, seed: int, zipf_s: float | None = None):
    g = _gen(seed)
    logits = torch.randn((T, E), generator=g)
    if zipf_s is not None:
        perm = torch.randperm(E, generator=g)
        ranks = torch.empty(E)
        ranks[perm] = torch.arange(1, E + 1, dtype=torch.float32)
        p = ranks.pow(-zipf_s)
        p = p / p.sum()
        logits = logits + torch.log(p)[None, :]
    return route(logits, k)


def make_hidden(T: int, H: int, seed: int, std: float = 1.0) -> torch.Tensor:
    g = _gen(seed)
    return (std * torch.randn((T, H), generator=g)).to(torch.bfloat16)


def make_norm_weight(H: int, seed: int) -> torch.Tensor:
    g = _gen(seed)
    return (1.0 + 0.1 * torch.randn((H,), generator=g)).to(torch.bfloat16)


def rmsnorm_256(seed: int = 0):
    g = _gen(seed)
    x = torch.randn((256, H_DG), generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn((H_DG,), generator=g)).to(torch.bfloat16)
    return x, w, 1e-6


def rmsnorm_32k(seed: int = 1, rows: int = 32768):
    g = _gen(seed)
    x = 2.0 * torch.randn((rows, H_DG), generator=g)
    out = torch.rand((rows, H_DG), generator=g) < 1e-3
    x = torch.where(out, x * 50.0, x).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn((H_DG,), generator=g)).to(torch.bfloat16)
    qk = torch.randn((256 * 16, 256), generator=g).to(torch.bfloat16)
    qk_w = (1.0 + 0.1 * torch.randn((256,), generator=g)).to(torch.bfloat16)
    return x, w, qk, qk_w, 1e-6


def layer_inputs(T: int, seed: int, zipf_s: float | None = None, E: int = E_DG, k: int = TOPK_DG,
                 H: int = H_DG):
    """hidden bf16 [T,H], norm weight bf16 [H], routing (ids, weights)."""
    g = _gen(seed)
    x = torch.randn((T, H), generator=g).to(torch.bfloat16)
    w = (1.0 + 0.1 * torch.randn((H,), generator=g)).to(torch.bfloat16)
    ids, wts = make_routing(T, E, k, seed + 1000, zipf_s)
    return x, w, ids, wts
