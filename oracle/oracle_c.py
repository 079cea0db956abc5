"""ctypes loader for oracle/liboracle.so (test infrastructure only)."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return os.path.join(_HERE, "liboracle.so")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.orc_combine.argtypes = [p, p, p, i64, i64, i64, ctypes.c_int, p, p]
        L.orc_combine.restype = ctypes.c_int
        L.orc_moe_align.argtypes = [p, i64, i64, i64, p, p, p]
        L.orc_moe_align.restype = ctypes.c_int
        L.orc_philox_first.argtypes = [p, i64, ctypes.c_uint32, ctypes.c_uint32, p]
        L.orc_philox_first.restype = None
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def combine(out3_f16: np.ndarray, inv: np.ndarray, topk_w: np.ndarray, out_bf16: bool = True):
    """Returns (y bits uint16 [T,H], y fp32 [T,H])."""
    out3 = np.ascontiguousarray(out3_f16, dtype=np.float16).view(np.uint16)
    inv = np.ascontiguousarray(inv, dtype=np.int64)
    w = np.ascontiguousarray(topk_w, dtype=np.float32)
    T, tk = w.shape
    H = out3.shape[1]
    y = np.empty((T, H), dtype=np.uint16)
    yf = np.empty((T, H), dtype=np.float32)
    rc = lib().orc_combine(_ptr(out3), _ptr(inv), _ptr(w), T, tk, H, int(out_bf16), _ptr(y), _ptr(yf))
    assert rc == 0
    return y, yf


def moe_align(topk_ids: np.ndarray, block_m: int, E: int):
    ids = np.ascontiguousarray(topk_ids, dtype=np.int64).reshape(-1)
    Nexp = ids.size
    max_blocks = (Nexp + block_m - 1) // block_m + E
    cap = max_blocks * block_m
    sorted_rows = np.empty(cap, dtype=np.int64)
    expert_ids = np.empty(max_blocks, dtype=np.int64)
    inv = np.empty(Nexp, dtype=np.int64)
    rc = lib().orc_moe_align(_ptr(ids), Nexp, E, block_m, _ptr(sorted_rows), _ptr(expert_ids), _ptr(inv))
    if rc == 2:
        raise IndexError("moe_align: negative expert id")
    assert rc == 0
    return sorted_rows, expert_ids, cap, inv


def philox_first(ctr: np.ndarray, k0: int, k1: int) -> np.ndarray:
    """First Philox4x32-10 output word for counters (c, 0, 0, 0), key (k0, k1)."""
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    out = np.empty_like(c)
    lib().orc_philox_first(_ptr(c), c.size, k0 & 0xFFFFFFFF, k1 & 0xFFFFFFFF, _ptr(out))
    return out
