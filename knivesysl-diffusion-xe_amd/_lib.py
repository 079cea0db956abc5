"""ctypes binding of libksl.so, the gfx950 HIP library (C ABI in include/ksl.h).

The library is the only compute path: if it is missing or does not load, every
entry point raises. There is no CPU or torch fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libksl.so")

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
ACT_GELU_TANH, ACT_SILU, ACT_NONE = 0, 1, 2
DN_LAYOUT_REF, DN_LAYOUT_TILED = 0, 1
ERR_ARG, ERR_SHAPE, ERR_ALIGN = 1, 2, 3
ERR_SCRATCH, ERR_RUNTIME = 6, 7
NOALLOC_SCRATCH_BYTES = 32 * 1024 * 1024
# int32 index of the one-launch FFN's error word in its ctl counters
FFN_ERROR_WORD = 64

_TORCH_TO_CODE = {
    torch.float32: DTYPE_F32,
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
}

# (name, argtypes, restype) of every exported symbol of include/ksl.h
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
SIGNATURES = {
    "ksl_version": ([], _I),
    "ksl_status_string": ([_I], ctypes.c_char_p),
    "ksl_rmsnorm": ([_P, _I, _P, _I, _P, _I, _I64, _I64, _I64, _I64, _F, _P], _I),
    "ksl_moe_align": ([_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P], _I),
    "ksl_moe_align_i32_capacity": ([_I64, _I64, _I64, _I64], _I64),
    "ksl_moe_align_i32": ([_P, _I64, _I64, _I64, _I64, _P, _P, _P, _P], _I),
    "ksl_moe_workspace_bytes": ([_I64, _I64, _I64, _I64, _I64], _SZ),
    "ksl_moe_w4a16_forward": ([_P, _I, _I64, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P,
                               _I64, _I64, _I64, _I64, _I64, _I, _P, _I, _I64, _P, _SZ, _P], _I),
    "ksl_moe_route": ([_P, _I64, _I64, _I64, _P, _P, _P, _P, _I, _I64, _I64, _P, _P], _I),
    "ksl_moe_gateup_act": ([_P, _P, _P, _I64, _I64, _P, _P, _P, _I64, _I64, _I64, _I, _P, _P], _I),
    "ksl_moe_down": ([_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _I, _P], _I),
    "ksl_quantize_w4": ([_P, _I, _I64, _I64, _I64, _P, _P, _P, _P], _I),
    "ksl_moe_down_lds_bytes": ([_I64, _I64, _I64, _I64], _SZ),
    "ksl_moe_unshuffle_ns_down": ([_P, _I64, _I64, _I64, _P, _P], _I),
    "ksl_moe_preshuffle_ns_down": ([_P, _I64, _I64, _I64, _P, _P], _I),
    "ksl_dequant_w4": ([_P, _P, _P, _I64, _I64, _I64, _P, _P], _I),
    "ksl_moe_repack_down_bytes": ([_I64, _I64, _I64], _SZ),
    "ksl_moe_repack_down": ([_P, _P, _P, _I64, _I64, _I64, _P, _P], _I),
    "ksl_moe_combine": ([_P, _P, _P, _I, _I64, _I64, _I64, _P, _I, _I64, _P], _I),
    "ksl_moe_combine_v1": ([_P, _P, _P, _I, _I64, _I64, _I64, _P, _I, _I64, _P], _I),
    "ksl_moe_combine_stock": ([_P, _P, _P, _I64, _P, _I, _I64, _I64, _I64, _P, _I, _I64, _P], _I),
    "ksl_moe_act_to_down_order": ([_P, _I64, _I64, _P, _P], _I),
    "ksl_moe_layer_forward": ([_P, _I, _I64, _P, _I, _F, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P,
                               _I64, _I64, _I64, _I64, _I64, _I, _P, _I, _I64, _P, _SZ, _P], _I),
    "ksl_moe_layer_forward_noalloc": ([_P, _I, _I64, _P, _I, _F, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P,
                                       _I64, _I64, _I64, _I64, _I64, _I, _P, _I, _I64, _P], _I),
    "ksl_moe_layer_route": ([_P, _I64, _I64, _I64, _P, _P, _P, _P, _I, _I64, _P, _I, _F, _I64, _P, _P, _SZ, _P], _I),
    "ksl_moe_route_scratch_bytes": ([_I64, _I64, _I64], _SZ),
    "ksl_moe_router": ([_P, _I, _I64, _P, _P, _P, _I, _F, _I64, _I64, _I64, _I64, _P, _P, _P, _P], _I),
    "ksl_moe_combine_post": ([_P, _P, _P, _I, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _F, _P, _F,
                              _P, _I, _P, _I64, _P], _I),
    "ksl_moe_block_forward": ([_P, _I64, _P, _F, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I, _P, _P,
                               _I64, _I64, _I64, _I64, _I64, _I, _P, _I64, _P, _F, _P, _F, _P, _I,
                               _P, _I64, _P, _SZ, _P], _I),
    "ksl_moe_ffn_ctl_bytes": ([_I64], _SZ),
    "ksl_moe_ffn": ([_P, _P, _P, _I64, _I64, _P, _P, _I64, _I64, _I64, _I, _P, _P, _P, _P], _I),
    "ksl_moe_ffn_set_wait_limit": ([_I64, _I], _I),
    "ksl_moe_pack_gateup_bytes": ([_I64, _I64, _I64], _SZ),
    "ksl_moe_pack_gateup": ([_P, _P, _P, _I64, _I64, _I64, _P, _P], _I),
    "ksl_moe_pack_down_bytes": ([_I64, _I64, _I64], _SZ),
    "ksl_moe_pack_down": ([_P, _P, _P, _I, _I64, _I64, _I64, _P, _P], _I),
    "ksl_entropy": ([_P, _I, _I64, _I64, _I64, _P, _P], _I),
    "ksl_gumbel_argmax": ([_P, _I, _I64, _I64, _I64, _I64, _P, _P, _P], _I),
    "ksl_sample_step": ([_P, _I, _I64, _I64, _I64, _I64, _P, _P, _P, _P], _I),
}

_lock = threading.Lock()
_lib = None


class KslError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load libksl.so (built by build.py). Raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise KslError(
                    f"{LIB_PATH} is missing: build it with `python knivesysl-diffusion-xe_amd/build.py` "
                    "(there is no fallback path)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (argtypes, restype) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = restype
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().ksl_status_string(rc).decode()
        raise KslError(f"{what} failed: {msg} (status {rc})")


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _TORCH_TO_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    if not t.is_cuda:
        raise ValueError("tensor must be on a GPU (device 'cuda')")
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())
