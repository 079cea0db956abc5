"""W4A16 128-expert fused MoE forward on gfx950 — drop-in for kernels/fused_moe_w4_v2.py.

  fused_moe_w4_v2(hidden, exp, topk_ids, topk_w) -> Tensor   (kernels/fused_moe_w4_v2.py:319-371)

`exp` is the reference's duck-typed experts module (kernels/pack_experts.py:96-97):
  gu_q uint8 [E, 2I, H/2], gu_s / gu_z fp16 [E, 2I, H/128]   (gate rows 0..I-1, up rows I..2I-1)
  dn_q uint8 [E, H, I/2],  dn_s / dn_z fp16 [E, H, I/64]
  act_fn                                                       (tanh-GELU or SiLU)
Packed format (kernels/w4a16.py:19-48): byte j of a row = q[2j] | q[2j+1] << 4,
W = fp16((q - zero) * scale) per (row, group).

One C call launches four kernels on the current stream, with no host sync:
routing metadata + fp16 activation copy, grouped gate/up GEMM with the
activation in the epilogue, grouped down GEMM, fixed-order top-k combine.
The combine is a fixed fp32 FMA chain over the top-k slots (no atomics), so
the output is bit-identical run to run.

Differences from the reference, on purpose:
- SiLU-gated experts are supported next to tanh-GELU (the reference asserts
  tanh-GELU, :291-308, :332).
- The preshuffled down pack (MOE_NS, :180-245) is not run as such.
  enable_ns_down (:200-206) installs, at load time, the down layout this
  build's kernel streams instead: the tiled layout, the same nibbles
  regrouped in the order the down kernel loads them (enable_tiled_down,
  flagged by `dn_tiled`). A module that arrives flagged `dn_ns` (an NS pack
  made elsewhere) is converted on its first forward. Results are those of
  the plain pack. preshuffle_T_dn still writes the NS bytes exactly (for
  checkpoints or comparisons).
- zero-points must be integers in [0, 15] (what quantize_w4 writes,
  kernels/w4a16.py:28). check_zero_points verifies it with one host sync;
  the load-time helpers (enable_tiled_down, enable_pack, pack_experts'
  repack_experts and load helpers) call it. A module none of them saw is
  checked on its first forward outside graph capture; under capture the
  check is skipped (no host sync is allowed there).
"""
from __future__ import annotations

import os
import weakref

import torch

from . import _lib

_TANH_GELU_NAMES = ("gelu_pytorch_tanh", "gelu_new", "gelu_tanh", "quick_gelu_tanh")  # :291
_SILU_NAMES = ("silu", "swish", "SiLU", "SiLUActivation")


def hidden_device(exp):
    """kernels/fused_moe_w4_v2.py:311-316."""
    for b in ("gu_s", "gu_q"):
        t = getattr(exp, b, None)
        if t is not None:
            return t.device
    return "cpu"


@torch.no_grad()
def moe_align_cuda(topk_ids: torch.Tensor, block_m: int, E: int):
    """kernels/fused_moe_w4_v2.py:46-76: (a_row int32[cap], expert_ids
    int32[cap // block_m], cap, inv int32[T*topk]) in one launch
    (ksl_moe_align_i32). cap follows the reference's capacity rule, padding
    slots hold T and padding blocks E. Every id must be a real expert in
    [0, E), as the reference requires; MOE_VALIDATE=1 adds the reference's
    synchronous range assert (:54-56)."""
    if topk_ids.dim() != 2:
        raise ValueError("topk_ids must be [T, topk]")
    if os.environ.get("MOE_VALIDATE") == "1":
        mn, mxv = int(topk_ids.min()), int(topk_ids.max())
        assert 0 <= mn and mxv < E, f"moe_align_cuda: ids must be in [0,{E}); got [{mn},{mxv}]"
    T, tk = topk_ids.shape
    block_m, E = int(block_m), int(E)
    if block_m <= 0 or E <= 0:
        raise ValueError("block_m and E must be positive")
    if E > 512:
        raise ValueError("E > 512 experts is not supported")
    if not topk_ids.is_cuda:
        raise ValueError("topk_ids must be on the GPU")
    lib = _lib.load()
    cap = int(lib.ksl_moe_align_i32_capacity(T, tk, E, block_m))
    dev = topk_ids.device
    ids = topk_ids.to(torch.int64).contiguous()
    a_row = torch.empty(cap, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(cap // block_m, dtype=torch.int32, device=dev)
    inv = torch.empty(T * tk, dtype=torch.int32, device=dev)
    rc = lib.ksl_moe_align_i32(_lib.ptr(ids), T, tk, E, block_m, _lib.ptr(a_row), _lib.ptr(expert_ids),
                               _lib.ptr(inv), _lib.stream_of(ids))
    _lib.check(rc, "ksl_moe_align_i32")
    return a_row, expert_ids, cap, inv


def _act_code(fn) -> int | None:
    name = (getattr(fn, "__name__", None) or type(fn).__name__) if fn is not None else None
    if name is None:
        return None
    # as the reference (kernels/fused_moe_w4_v2.py:297): a known tanh-GELU name or
    # any name containing "gelu" selects the tanh-GELU epilogue
    if name in _TANH_GELU_NAMES or "gelu" in str(name).lower():
        return _lib.ACT_GELU_TANH
    if name in _SILU_NAMES or "silu" in str(name).lower() or "swish" in str(name).lower():
        return _lib.ACT_SILU
    # numeric probe (kernels/fused_moe_w4_v2.py:299-302), on the CPU
    x = torch.tensor([-1.0, 0.0, 0.5, 2.0], dtype=torch.float32)
    try:
        out = fn(x).float()
    except Exception:
        return None
    gelu = 0.5 * x * (1.0 + torch.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))
    if torch.allclose(out, gelu, atol=1e-3):
        return _lib.ACT_GELU_TANH
    if torch.allclose(out, torch.nn.functional.silu(x), atol=1e-3):
        return _lib.ACT_SILU
    return None


def _check_act(exp) -> bool:
    """One-time guard (kernels/fused_moe_w4_v2.py:294-308): the epilogue is
    tanh-GELU or SiLU; the module's act_fn must be one of them."""
    fn = getattr(exp, "act_fn", None)
    code = _act_code(fn)
    name = (getattr(fn, "__name__", None) or type(fn).__name__) if fn is not None else None
    assert code is not None, (
        f"fused_moe_w4_v2 supports tanh-GELU and SiLU epilogues but this module's act_fn is {name!r}.")
    exp._ksl_act = code
    exp._act_checked = True
    return True


class _WeakValueCache(dict):
    """A cache for enable_tiled_down whose entries hold the converted tensor
    weakly: an entry lives as long as some module still uses the tensor (its
    sources are checked by identity, as in any cache given to it)."""

    def get(self, key, default=None):
        entry = super().get(key)
        if entry is None:
            return default
        refs, vref = entry
        value = vref()
        if value is None:
            del self[key]
            return default
        return refs, value

    def __setitem__(self, key, entry):
        refs, value = entry
        super().__setitem__(key, (refs, weakref.ref(value)))


# Modules still in the MOE_NS down layout at their first forward (no load-time
# repack ran) are converted there, through this process-wide cache, so the
# encoder and decoder experts of a layer that share one dn_q
# (kernels/load_w4_checkpoint.py:56-59) keep sharing one converted tensor.
_NS_FIRST_FORWARD = _WeakValueCache()


def _check_weights(exp, E, H, I) -> None:
    """Shapes, dtypes, contiguity and device of the six buffers (host-side
    only, no sync); a module in the MOE_NS down layout is converted first (one
    allocation and one repack launch, once per shared buffer; repack_experts
    or enable_ns_down at load time avoids that inside the first forward)."""
    if getattr(exp, "_ksl_weights_checked", False):
        return
    if getattr(exp, "dn_ns", False):
        enable_tiled_down(exp, _NS_FIRST_FORWARD)
    spec = {
        "gu_q": ((E, 2 * I, H // 2), torch.uint8),
        "gu_s": ((E, 2 * I, H // 128), torch.float16),
        "gu_z": ((E, 2 * I, H // 128), torch.float16),
        "dn_q": ((E, H, I // 2), torch.uint8),
        "dn_s": ((E, H, I // 64), torch.float16),
        "dn_z": ((E, H, I // 64), torch.float16),
    }
    for name, (shape, dt) in spec.items():
        t = getattr(exp, name)
        if tuple(t.shape) != shape:
            raise ValueError(f"exp.{name} has shape {tuple(t.shape)}, expected {shape}")
        if t.dtype != dt:
            raise TypeError(f"exp.{name} has dtype {t.dtype}, expected {dt}")
        if not t.is_contiguous():
            raise ValueError(f"exp.{name} must be contiguous")
        if not t.is_cuda:
            raise ValueError(f"exp.{name} must be on the GPU")
    exp._ksl_weights_checked = True


@torch.no_grad()
def check_zero_points(exp) -> None:
    """Raise unless every zero-point of exp (gu_z, dn_z) is an integer in
    [0, 15], the kernels' contract. One host sync; once per module (flagged)."""
    if getattr(exp, "_ksl_zeros_checked", False):
        return
    for name in ("gu_z", "dn_z"):
        z = getattr(exp, name)
        ok = bool(((z == z.round()) & (z >= 0) & (z <= 15)).all().item())
        if not ok:
            raise ValueError(f"exp.{name}: zero-points must be integers in [0, 15]")
    exp._ksl_zeros_checked = True


def check_zero_points_once(exp) -> None:
    """check_zero_points on a module that no load-time helper has checked,
    unless the current stream is being captured into a graph (a host sync
    is not allowed there: the check is then left to a later eager call)."""
    if getattr(exp, "_ksl_zeros_checked", False):
        return
    if torch.cuda.is_current_stream_capturing():
        return
    check_zero_points(exp)


@torch.no_grad()
def unshuffle_ns_down(ns_q: torch.Tensor) -> torch.Tensor:
    """The MOE_NS down pack [E, I/2, H] (kernels/fused_moe_w4_v2.py:187-197)
    -> a new [E, H, I/2] tensor in the reference layout (ksl_moe_unshuffle_ns_down)."""
    E, Ih, H = ns_q.shape
    if not ns_q.is_cuda or ns_q.dtype != torch.uint8 or not ns_q.is_contiguous():
        raise ValueError("the NS down pack must be a contiguous uint8 tensor on the GPU")
    out = torch.empty(E, H, Ih, dtype=torch.uint8, device=ns_q.device)
    rc = _lib.load().ksl_moe_unshuffle_ns_down(_lib.ptr(ns_q), E, H, 2 * Ih, _lib.ptr(out), _lib.stream_of(ns_q))
    _lib.check(rc, "ksl_moe_unshuffle_ns_down")
    return out


def _same_device(dev, **tensors) -> None:
    """The kernels dereference every pointer on `dev`: a tensor elsewhere
    (a CPU routing tensor, a module on another GPU) is refused here."""
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise ValueError(f"{name} is on {t.device}, the activations on {dev}")


def _cache_get(cache: dict | None, key, *sources):
    """The cached value for key if every source tensor it was made from is
    still the very tensor given (a freed tensor's address can be reused by a
    new allocation: the key alone would bind another module's data)."""
    if cache is None:
        return None
    entry = cache.get(key)
    if entry is None:
        return None
    refs, value = entry
    if len(refs) != len(sources) or any(r() is not src for r, src in zip(refs, sources)):
        del cache[key]
        return None
    return value


def _cache_put(cache: dict | None, key, value, *sources) -> None:
    if cache is not None:
        cache[key] = (tuple(weakref.ref(src) for src in sources), value)


def dn_layout(exp) -> int:
    """The C ABI's down layout code of exp. A tiled module's dn_q must be the
    front of a buffer written by ksl_moe_repack_down (the down kernel reads
    the pair table behind it): checked here on the host, so that a copy of
    the bare [E, H, I/2] view (which drops the table) is refused."""
    if not getattr(exp, "dn_tiled", False):
        return _lib.DN_LAYOUT_REF
    q = exp.dn_q
    E, H, Ih = q.shape
    need = int(_lib.load().ksl_moe_repack_down_bytes(E, H, 2 * Ih))
    st = q.untyped_storage()
    have = st.nbytes() - (q.data_ptr() - st.data_ptr())
    if have < need:
        raise ValueError("exp.dn_q is flagged dn_tiled but holds no pair table behind its weights "
                         "(a copy of the tiled view?): re-run enable_tiled_down on the reference layout")
    return _lib.DN_LAYOUT_TILED


@torch.no_grad()
def tiled_down(dn_q: torch.Tensor, dn_s: torch.Tensor, dn_z: torch.Tensor) -> torch.Tensor:
    """dn_q [E, H, I/2] uint8 (reference layout) with its scales and
    zero-points fp16 [E, H, I/64] -> a new [E, H, I/2] tensor in the tiled
    layout, the front of a buffer whose tail holds the (scale, zero) pair
    table the down kernel streams (ksl_moe_repack_down)."""
    E, H, Ih = dn_q.shape
    if not dn_q.is_cuda or dn_q.dtype != torch.uint8 or not dn_q.is_contiguous():
        raise ValueError("dn_q must be a contiguous uint8 tensor on the GPU")
    for name, t in (("dn_s", dn_s), ("dn_z", dn_z)):
        if t.dtype != torch.float16 or tuple(t.shape) != (E, H, 2 * Ih // 64) or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float16 [E, H, I/64] tensor")
        if t.device != dn_q.device:
            raise ValueError(f"{name} is on {t.device}, dn_q on {dn_q.device}")
    lib = _lib.load()
    buf = torch.empty(int(lib.ksl_moe_repack_down_bytes(E, H, 2 * Ih)), dtype=torch.uint8, device=dn_q.device)
    rc = lib.ksl_moe_repack_down(_lib.ptr(dn_q), _lib.ptr(dn_s), _lib.ptr(dn_z), E, H, 2 * Ih, _lib.ptr(buf),
                                 _lib.stream_of(dn_q))
    _lib.check(rc, "ksl_moe_repack_down")
    return buf[: E * H * Ih].view(E, H, Ih)


def enable_tiled_down(exp, cache: dict | None = None):
    """Swap exp.dn_q to the tiled layout in place (idempotent via the dn_tiled
    flag), as the reference's enable_ns_down swaps in its preshuffled pack
    (kernels/fused_moe_w4_v2.py:200-206); a module already in that NS layout
    (dn_ns) is converted from it. Checks the zero-points (check_zero_points).
    `cache` maps an original buffer to its
    repacked tensor, so modules that share one dn_q (the encoder and decoder
    experts of a layer, kernels/load_w4_checkpoint.py:56-59) keep sharing one."""
    if getattr(exp, "dn_tiled", False):
        return exp
    srcs = (exp.dn_q, exp.dn_s, exp.dn_z)
    key = tuple(t.data_ptr() for t in srcs) + (str(exp.dn_q.device), bool(getattr(exp, "dn_ns", False)))
    t = _cache_get(cache, key, *srcs)
    if t is None:
        ref = unshuffle_ns_down(exp.dn_q) if getattr(exp, "dn_ns", False) else exp.dn_q
        t = tiled_down(ref, exp.dn_s, exp.dn_z)
        _cache_put(cache, key, t, *srcs)
    exp.dn_q = t
    exp.dn_ns = False
    exp.dn_tiled = True
    check_zero_points(exp)
    return exp


@torch.no_grad()
def preshuffle_T_dn(qpacked: torch.Tensor, BK: int = 64) -> torch.Tensor:
    """kernels/fused_moe_w4_v2.py:186-197: the down pack [E, N, K/2] in the
    reference layout -> the MOE_NS pack [E, K/2, N] (within each BK = 64 chunk
    byte j = q[k0 + j] | q[k0 + 32 + j] << 4, transposed), byte for byte, by
    one launch (ksl_moe_preshuffle_ns_down)."""
    if BK != 64:
        raise ValueError("the MOE_NS pack is defined for BK = 64 (the down group size)")
    E, N, Kh = qpacked.shape
    if not qpacked.is_cuda or qpacked.dtype != torch.uint8 or not qpacked.is_contiguous():
        raise ValueError("qpacked must be a contiguous uint8 tensor on the GPU")
    out = torch.empty(E, Kh, N, dtype=torch.uint8, device=qpacked.device)
    rc = _lib.load().ksl_moe_preshuffle_ns_down(_lib.ptr(qpacked), E, N, 2 * Kh, _lib.ptr(out),
                                                _lib.stream_of(qpacked))
    _lib.check(rc, "ksl_moe_preshuffle_ns_down")
    return out


def enable_ns_down(exp, cache: dict | None = None):
    """kernels/fused_moe_w4_v2.py:200-206: the load-time switch to the faster
    down pack, in place and idempotent. The reference installs its MOE_NS
    pack for its NS kernel; this build installs the layout its own down kernel
    streams (enable_tiled_down: the same nibbles regrouped, the plain pack's
    results), with `cache` keeping shared buffers shared. A module whose dn_q
    already is an NS pack (dn_ns) is converted from it."""
    return enable_tiled_down(exp, cache)


@torch.no_grad()
def pack_weights(exp) -> tuple[torch.Tensor, torch.Tensor]:
    """The experts' gate/up and down weights in the pack layout of the
    one-launch expert FFN (ksl_moe_pack_gateup / ksl_moe_pack_down): new
    uint8 tensors holding the same nibbles, scales and zero-points."""
    E, twoI, Hh = exp.gu_q.shape
    H, I = 2 * Hh, twoI // 2
    _check_weights(exp, E, H, I)
    check_zero_points(exp)
    lib = _lib.load()
    st = _lib.stream_of(exp.gu_q)
    gu = torch.empty(int(lib.ksl_moe_pack_gateup_bytes(E, H, I)), dtype=torch.uint8, device=exp.gu_q.device)
    dn = torch.empty(int(lib.ksl_moe_pack_down_bytes(E, H, I)), dtype=torch.uint8, device=exp.gu_q.device)
    _lib.check(lib.ksl_moe_pack_gateup(_lib.ptr(exp.gu_q), _lib.ptr(exp.gu_s), _lib.ptr(exp.gu_z), E, H, I,
                                       _lib.ptr(gu), st), "ksl_moe_pack_gateup")
    _lib.check(lib.ksl_moe_pack_down(_lib.ptr(exp.dn_q), _lib.ptr(exp.dn_s), _lib.ptr(exp.dn_z), dn_layout(exp),
                                     E, H, I, _lib.ptr(dn), st), "ksl_moe_pack_down")
    return gu, dn


def enable_pack(exp, cache: dict | None = None):
    """Give exp the pack layout (exp.gu_pack, exp.dn_pack), with which the
    forwards of this package run gate/up and down as one launch for routings
    of at most 8192 rows (same results). The reference buffers stay for larger
    routings. Idempotent; `cache` keeps modules that share their buffers (the
    encoder and decoder experts of a layer, kernels/load_w4_checkpoint.py:56-59)
    sharing one pack."""
    if getattr(exp, "gu_pack", None) is not None and getattr(exp, "dn_pack", None) is not None:
        return exp
    srcs = (exp.gu_q, exp.dn_q)
    key = (exp.gu_q.data_ptr(), exp.dn_q.data_ptr(), str(exp.gu_q.device))
    t = _cache_get(cache, key, *srcs)
    if t is None:
        t = pack_weights(exp)
        _cache_put(cache, key, t, *srcs)
    exp.gu_pack, exp.dn_pack = t
    return exp


def pack_ptrs(exp):
    """(gu_pack, dn_pack) device pointers for the C forwards (NULL without a pack)."""
    return _lib.ptr(getattr(exp, "gu_pack", None)), _lib.ptr(getattr(exp, "dn_pack", None))


def moe_workspace(T: int, tk: int, E: int, H: int, I: int, device) -> torch.Tensor:
    nbytes = int(_lib.load().ksl_moe_workspace_bytes(T, tk, E, H, I))
    return torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)


@torch.no_grad()
def fused_moe_w4_v2(hidden: torch.Tensor, exp, topk_ids: torch.Tensor, topk_w: torch.Tensor,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    T, K = hidden.shape
    tk = topk_ids.shape[1]
    E, twoI, _ = exp.gu_q.shape
    I = twoI // 2
    assert K % 128 == 0, f"hidden dim {K} must be divisible by 128 (gate_up group)"
    assert I % 64 == 0, f"expert intermediate {I} must be divisible by 64 (down group)"
    assert getattr(exp, "_act_checked", False) or _check_act(exp), "unsupported activation"
    if not hasattr(exp, "_ksl_act"):
        _check_act(exp)
    _check_weights(exp, E, K, I)
    check_zero_points_once(exp)
    if topk_ids.shape[0] != T or tuple(topk_w.shape) != (T, tk):
        raise ValueError("topk_ids / topk_w must be [T, topk]")
    dev = hidden.device
    _same_device(dev, topk_ids=topk_ids, topk_w=topk_w, gu_q=exp.gu_q)
    if hidden.stride(1) != 1 or hidden.stride(0) % 8 != 0 or hidden.data_ptr() % 16 != 0:
        hidden = hidden.clone(memory_format=torch.contiguous_format)  # a fresh, aligned copy
    ids = topk_ids if topk_ids.dtype == torch.int64 else topk_ids.to(torch.int64)
    ids = ids.contiguous()
    w = topk_w.contiguous()
    out_dtype = hidden.dtype
    # the reference stores fp16 for any non-bf16 hidden (:260-263)
    y_dtype = torch.bfloat16 if out_dtype == torch.bfloat16 else torch.float16
    y = torch.empty(T, K, dtype=y_dtype, device=dev)
    if T == 0:
        return y.to(out_dtype)
    if workspace is None:
        workspace = moe_workspace(T, tk, E, K, I, dev)
    lib = _lib.load()
    rc = lib.ksl_moe_w4a16_forward(
        _lib.ptr(hidden), _lib.dtype_code(hidden.dtype), hidden.stride(0),
        _lib.ptr(ids), _lib.ptr(w), _lib.dtype_code(w.dtype),
        _lib.ptr(exp.gu_q), _lib.ptr(exp.gu_s), _lib.ptr(exp.gu_z),
        _lib.ptr(exp.dn_q), _lib.ptr(exp.dn_s), _lib.ptr(exp.dn_z), dn_layout(exp), *pack_ptrs(exp),
        T, tk, E, K, I, exp._ksl_act,
        _lib.ptr(y), _lib.dtype_code(y_dtype), y.stride(0),
        _lib.ptr(workspace), workspace.numel(), _lib.stream_of(hidden))
    _lib.check(rc, "ksl_moe_w4a16_forward")
    return y if y_dtype == out_dtype else y.to(out_dtype)
