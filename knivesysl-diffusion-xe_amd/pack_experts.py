"""Experts forward binding — drop-in for kernels/pack_experts.py.

  fused_experts_forward(self, hidden_states, top_k_index, top_k_weights)
                                                   (kernels/pack_experts.py:65-84)
is bound per DiffusionGemmaTextExperts module by the loader
(kernels/load_w4_checkpoint.py:83). As in the reference, MOE_V2 selects the
path: "1" the v2 forward (fused_moe_w4_v2), any other value the v1 forward
(fused_moe_w4, any act_fn). Unset: v2 when the module's activation is one the
v2 epilogue has (tanh-GELU or SiLU), else v1. (The reference's loader sets
MOE_V2=1 at import, kernels/load_w4_checkpoint.py:22, so its deployed path is
v2; unset it would run v1.) MOE_STATS=1 records the reference's routing probe
(the expert union at top-8/6/4/2 and the experts holding 80% of the routing
mass, :14-31, :69-78); dump_moe_stats() prints it.

  packed_experts_forward(self, hidden_states, top_k_index, top_k_weights)
                                                   (kernels/pack_experts.py:44-62)
the stock experts loop over the W4 linears: gate/up, act_fn(gate) * up, down,
then the stock expert-ordered index_add_ combine (ksl_moe_combine_stock).
GU_GS / DN_GS are the pack's group sizes (kernels/pack_experts.py:12).

repack_experts(model) is the load-time repack (after the loader binds the
packed buffers, kernels/load_w4_checkpoint.py:76-83): every experts module's
down weights go to the tiled layout the down kernel loads, once per buffer,
so the encoder and decoder modules that share a layer's tensors
(:56-59) keep sharing one repacked tensor.

pack_experts_module / pack_all_experts (kernels/pack_experts.py:87-122)
quantise a bf16 experts module in place with the GPU quantiser
(w4a16.quantize_w4): the six packed buffers, the tiled down layout, the
fused (or, with fused=False, the packed loop) forward bound.
"""
from __future__ import annotations

import collections
import os

import torch

from .fused_moe_w4 import expert_rows_forward, fused_moe_w4
from .fused_moe_w4_v2 import _act_code, enable_ns_down, enable_tiled_down, fused_moe_w4_v2
from .w4a16 import quantize_w4

GU_GS, DN_GS = 128, 64
EXPERT_BUFS = ("gu_q", "gu_s", "gu_z", "dn_q", "dn_s", "dn_z")  # kernels/load_w4_checkpoint.py:27

# routing probe records (MOE_STATS=1): per MoE forward the expert union at
# top-8/6/4/2, the experts holding 80% of the routing mass, the expert count
_MOE_ACC: dict = collections.defaultdict(list)


@torch.no_grad()
def _record_moe_stats(top_k_index: torch.Tensor, top_k_weights: torch.Tensor, num_experts: int) -> None:
    """kernels/pack_experts.py:69-78: one forward's routing statistics (a
    diagnostic: it synchronises the host)."""
    order = top_k_weights.argsort(dim=-1, descending=True)  # [:, :k] = the true top-k
    tis = torch.gather(top_k_index, -1, order)
    tk = top_k_index.shape[1]
    for k, key in ((8, "u8"), (6, "u6"), (4, "u4"), (2, "u2")):
        _MOE_ACC[key].append(int(tis[:, :min(k, tk)].unique().numel()))
    hist = torch.bincount(top_k_index.reshape(-1), minlength=num_experts).float()
    cum = torch.cumsum(torch.sort(hist, descending=True).values, 0) / hist.sum().clamp(min=1)
    _MOE_ACC["conc"].append(int((cum < 0.8).sum()) + 1)
    _MOE_ACC["E"].append(num_experts)


def dump_moe_stats() -> None:
    """kernels/pack_experts.py:19-31: print the routing probe's averages."""
    if not _MOE_ACC.get("u8"):
        return
    m = lambda x: sum(x) / len(x)  # noqa: E731
    E = _MOE_ACC["E"][0]
    u8, u6, u4, u2 = (m(_MOE_ACC[k]) for k in ("u8", "u6", "u4", "u2"))
    print(f"\n=== MoE ROUTING PROBE (n={len(_MOE_ACC['u8'])} MoE-layer-forwards, {E} experts) ===", flush=True)
    print(f"  expert UNION loaded per forward:  top-8={u8:.0f}  top-6={u6:.0f}  top-4={u4:.0f}  top-2={u2:.0f}"
          f"   (of {E})", flush=True)
    print(f"  MoE bandwidth vs top-8:  top-6={100 * u6 / u8:.0f}%  top-4={100 * u4 / u8:.0f}%  "
          f"top-2={100 * u2 / u8:.0f}%", flush=True)
    print(f"  experts holding 80% of routing mass: {m(_MOE_ACC['conc']):.0f}/{E}", flush=True)
    print("  VERDICT: dynamic-k moves tok/s IFF top-4 union << top-8 (concentrated). If ~equal -> "
          "coupon-collector, no BW win.", flush=True)


def _use_v2(self) -> bool:
    flag = os.environ.get("MOE_V2")
    if flag is not None:
        return flag == "1"
    return _act_code(getattr(self, "act_fn", None)) is not None


def fused_experts_forward(self, hidden_states, top_k_index, top_k_weights):
    """kernels/pack_experts.py:65-84: all experts in one grouped forward."""
    if os.environ.get("MOE_STATS"):
        _record_moe_stats(top_k_index, top_k_weights, self.gu_q.shape[0])
    if _use_v2(self):
        return fused_moe_w4_v2(hidden_states, self, top_k_index, top_k_weights)
    return fused_moe_w4(hidden_states, self, top_k_index, top_k_weights)


def packed_experts_forward(self, hidden_states, top_k_index, top_k_weights):
    """kernels/pack_experts.py:44-62: the stock DiffusionGemmaTextExperts
    forward with both linears reading the packed W4 buffers, and its combine:
    zeros in the hidden dtype, then per expert in ascending id
    index_add_((h * w).to(dtype)) over the expert's tokens."""
    return expert_rows_forward(hidden_states, self, top_k_index, top_k_weights, combine="stock")


def repack_experts(model, verbose: bool = True) -> int:
    """Tile the down weights of every module holding the packed buffers
    (gu_q .. dn_z) in place; returns the number of modules. Idempotent."""
    cache: dict = {}
    n = 0
    for mod in model.modules():
        if hasattr(mod, "gu_q") and hasattr(mod, "dn_q"):
            enable_tiled_down(mod, cache)
            n += 1
    if verbose:
        print(f"[repack] {n} experts modules, {len(cache)} down buffers tiled")
    return n


@torch.no_grad()
def pack_experts_module(exp, free_bf16: bool = True, fused: bool = True, *, cache: dict | None = None):
    """Quantise one experts module in place (kernels/pack_experts.py:87-106):
    gate_up_proj [E, 2I, H] in groups of GU_GS along H, down_proj [E, H, I] in
    groups of DN_GS along I, as the six buffers the forwards read; the down
    weights then go to the tiled layout (enable_tiled_down, which also checks
    the zero-points; under MOE_NS=1 with MOE_V2=1 the reference's
    enable_ns_down switch, :101-103, installs the same layout), and the
    forward is bound: fused_experts_forward, or with fused=False the packed
    loop packed_experts_forward. free_bf16 drops the bf16 weights. `cache`
    keeps modules that share a tensor sharing its repacked copy."""
    gu = quantize_w4(exp.gate_up_proj.data, GU_GS)
    dn = quantize_w4(exp.down_proj.data, DN_GS)
    for name, t in zip(EXPERT_BUFS, gu + dn):
        exp.register_buffer(name, t, persistent=False)
    if free_bf16:
        exp.gate_up_proj = None
        exp.down_proj = None
    if os.environ.get("MOE_NS") == "1" and os.environ.get("MOE_V2") == "1":
        enable_ns_down(exp, cache)
    else:
        enable_tiled_down(exp, cache)
    fwd = fused_experts_forward if fused else packed_experts_forward
    exp.forward = fwd.__get__(exp, exp.__class__)
    return exp


@torch.no_grad()
def pack_all_experts(model, free_bf16: bool = True, verbose: bool = True) -> int:
    """pack_experts_module on every module with bf16 expert weights
    (gate_up_proj and down_proj, kernels/pack_experts.py:109-122)."""
    n, gu_elems, dn_elems = 0, 0, 0
    for mod in model.modules():
        gp, dp = getattr(mod, "gate_up_proj", None), getattr(mod, "down_proj", None)
        if isinstance(gp, torch.Tensor) and isinstance(dp, torch.Tensor) and gp.dim() == 3:
            gu_elems += gp.numel()
            dn_elems += dp.numel()
            pack_experts_module(mod, free_bf16)
            n += 1
    if verbose:
        gib = 2 ** 30
        print(f"[pack] {n} experts modules -> W4 (gate/up gs{GU_GS}, down gs{DN_GS}): "
              f"{2 * (gu_elems + dn_elems) / gib:.2f} GiB bf16 -> {(gu_elems + dn_elems) / 2 / gib:.2f} GiB W4",
              flush=True)
    return n
