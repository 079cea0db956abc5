"""The C ABI without a GPU: the library loads, exports every entry point that
include/ksl.h declares (and the ctypes table binds exactly those), and the
host-side parts (status strings, workspace sizing, argument validation that
returns before any device work) behave as documented."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from tests.conftest import ROOT, load_mod

HEADER = os.path.join(ROOT, "include", "ksl.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(ksl_[a-z0-9_]+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    names = _declared()
    for n in ("ksl_rmsnorm", "ksl_moe_align", "ksl_moe_w4a16_forward", "ksl_moe_layer_forward",
              "ksl_moe_gateup_act", "ksl_moe_down", "ksl_moe_combine", "ksl_moe_router", "ksl_moe_combine_post",
              "ksl_moe_block_forward", "ksl_moe_route_scratch_bytes", "ksl_version",
              "ksl_status_string"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = load_mod("_lib")
    path = lib.LIB_PATH
    assert os.path.exists(path), "build it first: python knivesysl-diffusion-xe_amd/build.py"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(ksl_[a-z0-9_]+)$", out, flags=re.M))
    declared = set(_declared())
    assert declared <= exported, f"declared but not exported: {sorted(declared - exported)}"
    assert set(lib.SIGNATURES) == declared, "ctypes table and header disagree"


@pytest.fixture(scope="module")
def L():
    return load_mod("_lib").load()


def test_host_only_calls(L):
    assert L.ksl_version() >= 1
    for code, word in ((0, "ok"), (1, "argument"), (2, "shape"), (3, "align")):
        assert word in L.ksl_status_string(code).decode().lower()
    assert L.ksl_status_string(99).decode()  # unknown codes still give text
    a = L.ksl_moe_workspace_bytes(256, 8, 128, 2816, 704)
    b = L.ksl_moe_workspace_bytes(512, 8, 128, 2816, 704)
    # sorted rows, offsets, inv, a16, out2, out3 at least
    assert a >= 256 * 8 * (704 + 2816) * 2 + 256 * 2816 * 2
    assert b > a


def test_align_i32_capacity(L):
    """The moe_align_cuda capacity rule (kernels/fused_moe_w4_v2.py:59-64) against
    the oracle's, over block sizes and the rows < experts branch."""
    from oracle import moe_oracle as mo
    for T, tk, E, bm in ((256, 8, 128, 32), (256, 8, 128, 16), (3, 2, 64, 16), (1, 1, 512, 64),
                         (100, 8, 128, 1), (0, 8, 128, 32), (7, 3, 8, 5)):
        ids = np.zeros((T, tk), dtype=np.int64)
        assert L.ksl_moe_align_i32_capacity(T, tk, E, bm) == mo.moe_align_cuda(ids, bm, E)[2]
    assert L.ksl_moe_align_i32_capacity(4, 2, 0, 32) == -1


def test_route_scratch_bytes(L):
    # block counts of the multi-block routing: ceil(T*topk / 1024) * E int32, none up to 4096 rows
    assert L.ksl_moe_route_scratch_bytes(512, 8, 128) == 0
    assert L.ksl_moe_route_scratch_bytes(513, 8, 128) == 5 * 128 * 4
    assert L.ksl_moe_route_scratch_bytes(8192, 8, 128) == 64 * 128 * 4
    assert L.ksl_moe_route_scratch_bytes(-1, 8, 128) == 0
    # the fused forward's workspace holds them after out3
    base = L.ksl_moe_workspace_bytes(512, 8, 128, 2816, 704)
    assert L.ksl_moe_workspace_bytes(513, 8, 128, 2816, 704) >= base + 5 * 128 * 4


def test_validation_returns_before_device_work(L):
    P = ctypes.c_void_p
    fake = P(1 << 20)  # never dereferenced: every call below fails its checks first
    null = P(0)
    # rows == 0 is a no-op, even with null pointers
    assert L.ksl_rmsnorm(null, 2, null, 2, null, 2, 0, 128, 128, 128, 1e-6, null) == 0
    assert L.ksl_rmsnorm(null, 2, null, 2, null, 2, 4, 128, 128, 128, 1e-6, null) == 1     # null x
    assert L.ksl_rmsnorm(fake, 7, null, 2, fake, 2, 4, 128, 128, 128, 1e-6, null) == 1     # bad dtype
    # gate/up: null pointers, then H not a multiple of 128, then misalignment
    assert L.ksl_moe_gateup_act(null, fake, fake, 256, 8, fake, fake, fake, 128, 2816, 704, 1, fake, null) == 1
    assert L.ksl_moe_gateup_act(fake, fake, fake, 256, 8, fake, fake, fake, 128, 2800, 704, 1, fake, null) == 2
    assert L.ksl_moe_gateup_act(P((1 << 20) + 8), fake, fake, 256, 8, fake, fake, fake, 128, 2816, 704, 1, fake,
                                null) == 3
    # down: I not a multiple of 64, I above 1024
    assert L.ksl_moe_down(fake, fake, fake, fake, fake, 128, 2816, 700, 2048, fake, 0, null) == 2
    assert L.ksl_moe_down(fake, fake, fake, fake, fake, 128, 2816, 1088, 2048, fake, 0, null) == 2
    assert L.ksl_moe_down(fake, fake, fake, fake, fake, 128, 2816, 704, 2048, fake, 7, null) == 1   # unknown layout
    assert L.ksl_moe_down(fake, fake, fake, fake, fake, 128, 2816, 704, -1, fake, 0, null) == 2
    assert L.ksl_moe_down(fake, fake, fake, fake, fake, 128, 2816, 704, 2048, P((1 << 20) + 4), 0, null) == 3  # out3 % 8
    assert L.ksl_moe_down(fake, fake, fake, fake, fake, 128, 2816, 704, 2048, P((1 << 20) + 8), 0, null) == 3  # out3 % 16
    # repack: shapes, in-place refused, alignment
    assert L.ksl_moe_repack_down(fake, fake, fake, 128, 2816, 700, P((1 << 21)), null) == 2
    assert L.ksl_moe_repack_down(fake, fake, fake, 128, 2816, 704, fake, null) == 1
    assert L.ksl_moe_repack_down(P((1 << 20) + 8), fake, fake, 128, 2816, 704, P(1 << 21), null) == 3
    assert L.ksl_moe_repack_down(fake, P((1 << 20) + 1), fake, 128, 2816, 704, P(1 << 21), null) == 3  # dn_s % 2
    assert L.ksl_moe_repack_down_bytes(128, 2816, 704) == 128 * 2816 * 352 + 128 * 2816 * 11 * 4
    # align: E above the routing limit
    assert L.ksl_moe_align(fake, 4, 8, 4096, 32, fake, fake, fake, null) == 2


def test_router_rejects_bad_arguments_without_launching():
    """Argument checks of ksl_moe_router run on the host (no GPU needed)."""
    lib = load_mod("_lib")
    L = lib.load()
    P = ctypes.c_void_p
    fake, null = P(1 << 20), P(0)
    # probs is required (it holds the scores between the two launches)
    assert L.ksl_moe_router(fake, 2, 2816, fake, fake, fake, 2, 1e-6, 256, 2816, 128, 8, null, fake, fake, null) == 1
    # E not a multiple of 16, k > 16, H not a multiple of 32
    assert L.ksl_moe_router(fake, 2, 2816, fake, fake, fake, 2, 1e-6, 256, 2816, 120, 8, fake, fake, fake, null) == 2
    assert L.ksl_moe_router(fake, 2, 2816, fake, fake, fake, 2, 1e-6, 256, 2816, 128, 17, fake, fake, fake, null) == 2
    assert L.ksl_moe_router(fake, 2, 2800, fake, fake, fake, 2, 1e-6, 256, 2800, 128, 8, fake, fake, fake, null) == 2
    # T = 0 is a no-op
    assert L.ksl_moe_router(null, 2, 2816, null, null, null, 2, 1e-6, 0, 2816, 128, 8, null, null, null, null) == 0


def test_block_tail_entry_points_reject_bad_arguments_without_launching():
    """Argument checks of ksl_moe_combine_post / ksl_moe_block_forward run on the host."""
    L = load_mod("_lib").load()
    P = ctypes.c_void_p
    fake, null = P(1 << 20), P(0)
    odd = P((1 << 20) + 8)

    def post(T=256, tk=8, H=2816, h1=fake, res=fake, ls=null, ls_dt=2, wd=0, ys=2816, y=fake):
        return L.ksl_moe_combine_post(fake, fake, fake, wd, T, tk, H, h1, 2816, res, 2816, fake, 1e-6, fake, 1e-6,
                                      ls, ls_dt, y, ys, null)
    assert post(T=0, h1=null, res=null, y=null) == 0          # no-op
    assert post(res=null) == 1                                # residual required
    assert post(ls=fake, ls_dt=1) == 1                        # layer scalar fp32 or bf16 only
    assert post(wd=5) == 1                                    # unknown weight dtype
    assert post(H=2820) == 2 and post(H=8200, ys=8200) == 2   # H % 8, H <= 8192
    assert post(ys=2800) == 2                                 # stride below H
    assert post(y=odd) == 3                                   # misaligned output

    def block(T=256, H=2816, I=704, act=1, h1=fake, ws=null, wsb=0, layout=0):
        return L.ksl_moe_block_forward(fake, H, fake, 1e-6, fake, fake, 0, fake, fake, fake, fake, fake, fake, layout,
                                       null, null, T, 8, 128, H, I, act, h1, H, fake, 1e-6, fake, 1e-6, null, 2, fake, H,
                                       ws, wsb, null)
    assert block(I=700) == 2 and block(H=2800) == 2
    assert block(act=9) == 1
    assert block(layout=2) == 1
    assert block(h1=null) == 1
    assert block() == 5                                       # workspace missing
    assert block(T=0) == 0


def test_down_lds_sizing_fits_gfx950(L):
    """ksl_moe_down's dynamic LDS: the activation blocks of one 64-row chunk
    (4 M tiles x I/64 x 2 blocks of 1 KB) and each of the 8 waves' output
    staging (2 M tiles x 16 rows x 80 bytes), within gfx950's 160 KB over the
    corners of the contract (E <= 512, H <= 4096, I <= 1024) and device sizes
    from 1 to 1024 CUs; the largest at I = 1024."""
    worst = 0
    for E in (1, 8, 128, 256, 512):
        for H in (128, 256, 2816, 3072, 4096):
            for I in (64, 128, 512, 704, 768, 1024):
                for cus in (1, 80, 256, 304, 1024):
                    lds = L.ksl_moe_down_lds_bytes(E, H, I, cus)
                    assert lds == 4 * 2 * (I // 64) * 1024 + 8 * 2 * 16 * 80, (E, H, I, cus, lds)
                    assert lds <= 160 * 1024, (E, H, I, cus, lds)
                    worst = max(worst, lds)
    assert worst == 4 * 2 * 16 * 1024 + 8 * 2 * 16 * 80
    assert L.ksl_moe_down_lds_bytes(128, 4096, 1088, 256) == 0  # I above the contract
    assert L.ksl_moe_down_lds_bytes(128, 4096, 100, 256) == 0   # I % 64 != 0
