"""The down kernel's generated code, checked on the CPU.

ksl_moe_down streams each wave's weight tiles (with their scale / zero-point
pairs) into registers by ordinary loads, whose waits the compiler places,
reads its activations from LDS and sends its outputs through a per-wave LDS
staging area. The device assembly of csrc/moe_gemm.hip is
built with the library's flags and a few workgroups of down_kernel are run
through tests/gfx950_emu.py: every global, buffer and LDS access must stay in
its buffer (the weights, the tiled layout's trailing pair table, out2,
out3), and no address, stored value or MFMA operand may come from a register
whose load had not landed (the compiler's waits are checked, not assumed).
Shapes: the 256-token layer (one chunk, up to two M tiles), 1024 tokens (four
M tiles, several chunks per expert), a Zipf routing of 1024 tokens (experts of
a few to many chunks), and small / odd I (a 64-K tail group, the largest I).
Above 8192 routed rows a different kernel runs (moe_rbgemm.hip): ordinary
register loads for its weights, and inline-asm LDS reads of its activation
fragments, whose in-flight windows are checked below on the generated code."""
from __future__ import annotations

import importlib.util
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import gfx950_emu as emu  # noqa: E402

ROOT = os.path.dirname(HERE)
CSRC = os.path.join(ROOT, "knivesysl-diffusion-xe_amd", "csrc")


def _build_flags():
    spec = importlib.util.spec_from_file_location("ksl_build", os.path.join(ROOT, "knivesysl-diffusion-xe_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.HIPCC, mod.HIP_FLAGS


@pytest.fixture(scope="module")
def down_asm(tmp_path_factory):
    hipcc, flags = _build_flags()
    if not (os.path.exists(hipcc) or shutil.which(hipcc)):
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("asm") / "moe_gemm.s")
    res = subprocess.run([hipcc, *flags, "-w", "--cuda-device-only", "-S", os.path.join(CSRC, "moe_gemm.hip"),
                          "-o", out], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    return out


# The launch plan of csrc/moe_gemm.hip (plan_down, kDnWaves, kDnMaxMt)
# restated for the emulated launches.
NW, MAX_MT, CUS = 8, 4, 256


def _plan(E, H, I):
    G = I // 64
    te = H // 16
    nsplit = max(1, min(-(-CUS // E), te))
    tpw = -(-te // nsplit)
    nsplit = -(-te // tpw)
    return nsplit, tpw, MAX_MT * 2 * G * 1024 + NW * 2 * 16 * 80  # activations, then the waves' output staging


def _routing(E, T, tk, kind, seed):
    rng = np.random.default_rng(seed)
    if kind == "uniform":
        ids = np.stack([rng.permutation(E)[:tk] for _ in range(T)])
    else:
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        p /= p.sum()
        ids = np.stack([rng.choice(E, tk, replace=False, p=p) for _ in range(T)])
    return np.bincount(ids.ravel(), minlength=E)


CASES = [
    # E, H, I, T, tk, routing, layout (0 reference, 1 tiled), workgroups
    (128, 2816, 704, 256, 8, "uniform", 1, (0, 77, 255)),
    (128, 2816, 704, 1024, 8, "uniform", 0, (1, 128)),
    (128, 2816, 704, 1024, 8, "zipf", 1, (6, 7, 255)),
    (16, 256, 192, 64, 4, "uniform", 0, (0, 200)),
    (2, 64, 1024, 64, 2, "uniform", 1, (0, 7)),
]


@pytest.mark.parametrize("E,H,I,T,tk,routing,layout,wgs", CASES)
def test_down_kernel_addresses_and_register_flow(down_asm, E, H, I, T, tk, routing, layout, wgs):
    G = I // 64
    fn = f"_ZN3ksl12_GLOBAL__N_111down_kernelILi{G // 2}ELb{G % 2}ELi{layout}EEEvNS0_6DnArgsE"
    ins, labels = emu.load_kernel(down_asm, fn)
    counts = _routing(E, T, tk, routing, E + H + I)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    nrows = int(counts.sum())
    nsplit, tpw, lds = _plan(E, H, I)
    assert nrows <= 8192  # larger routings run the row-block kernels
    grid = E * nsplit
    bufs, base = {}, 0x7F0000000000

    def alloc(name, size):
        nonlocal base
        bufs[name] = (base, base + size)
        base += ((size + 0xFFFFF) // 0x100000 + 16) * 0x100000
        return bufs[name][0]

    p_out2 = alloc("out2", nrows * I * 2)
    p_off = alloc("offsets", (E + 1) * 4)
    # the tiled layout's buffer: the weights, then the (scale, zero) pair table
    p_q = alloc("dn_q", E * H * I // 2 + (E * H * G * 4 if layout == 1 else 0))
    p_s = alloc("dn_s", E * H * G * 2)
    p_z = alloc("dn_z", E * H * G * 2)
    p_out3 = alloc("out3", nrows * H * 2)
    p_karg = alloc("kernarg", 352)
    p_sz = p_q + E * H * I // 2 if layout == 1 else 0
    early = 1 if nrows >= E else 0
    # DnArgs (80 bytes), then the first hidden argument (the grid's block count)
    karg = struct.pack("<QQQQQQQiiiii", p_out2, p_off, p_q, p_s, p_z, p_out3, p_sz, H, I, nsplit, tpw, early)
    karg += b"\0" * (80 - len(karg))
    karg += struct.pack("<I", grid) + b"\0" * 60
    mem = {p_karg + k: struct.unpack("<I", karg[k:k + 4])[0] for k in range(0, len(karg), 4)}
    mem.update({p_off + 4 * e: int(offsets[e]) for e in range(E + 1)})
    checked = 0
    for wg in wgs:
        assert wg < grid
        shared = None
        for wave_id in range(NW):
            w = emu.Wave(mem, p_karg, wg, wave_id, bufs, lds)
            if shared is not None:
                w.lds = shared
            emu.run(ins, labels, w)
            shared = w.lds
            checked += w.accesses
            assert not w.errors, (wg, wave_id, w.errors[:4])
    assert checked > 0


SYNTHETIC = """synthetic:
	global_load_dwordx4 v[4:7], v[0:1], off
	v_mov_b64_e32 v[8:9], v[4:5]
	s_waitcnt vmcnt(0)
	global_load_dword v10, v[8:9], off
	s_endpgm
.Lfunc_end0:
"""


def test_emulator_flags_a_copied_in_flight_register(tmp_path):
    """The hazard the checks above exclude, planted in a four-line kernel: a
    loaded register copied before its wait and the copy used as an address."""
    path = tmp_path / "syn.s"
    path.write_text(SYNTHETIC)
    ins, labels = emu.load_kernel(str(path), "synthetic")
    buf = (0x7F0000000000, 0x7F0000100000)
    w = emu.Wave({}, 0x7F0000200000, 0, 0, {"buf": buf, "karg": (0x7F0000200000, 0x7F0000200100)}, 1024)
    w.v[0] = np.uint64(buf[0] & 0xFFFFFFFF) + np.arange(64, dtype=np.uint64) * np.uint64(16)
    w.v[1] = np.uint64(buf[0] >> 32)
    emu.run(ins, labels, w)
    assert any(e[0] == "POISONED ADDRESS load" for e in w.errors), w.errors


@pytest.mark.parametrize("layout", [0, 1])
def test_down_kernel_every_width(down_asm, layout):
    """Every instantiation of down_kernel (I = 64 .. 1024, with and without a
    64-K tail group) on a small routing: one workgroup each, same checks."""
    for G in range(1, 17):
        I = 64 * G
        test_down_kernel_addresses_and_register_flow(down_asm, 4, 128, I, 48, 2, "uniform", layout, (0, 5))


# ---- the row-block GEMMs (moe_rbgemm.hip): activation fragments read by asm
@pytest.fixture(scope="module")
def rb_asm(tmp_path_factory):
    hipcc, flags = _build_flags()
    if not (os.path.exists(hipcc) or shutil.which(hipcc)):
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("asm") / "moe_rbgemm.s")
    res = subprocess.run([hipcc, *flags, "-w", "--cuda-device-only", "-S", os.path.join(CSRC, "moe_rbgemm.hip"),
                          "-o", out], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    return out


def _codegen_check():
    spec = importlib.util.spec_from_file_location(
        "ksl_codegen_check", os.path.join(ROOT, "knivesysl-diffusion-xe_amd", "codegen_check.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _ahead_windows(lines):
    return _codegen_check().ahead_windows(lines)


def test_rb_gemm_ahead_reads_stay_untouched_in_flight(rb_asm):
    """Every row-block kernel instance (gate/up and down, both activations and
    both weight layouts): each asm LDS read of the next M tile's activation
    fragment keeps its four destination registers untouched, with no branch,
    until the s_waitcnt lgkmcnt(0) that retires it; seven such reads per
    32-K step of the full-block path."""
    cc = _codegen_check()
    asm = open(rb_asm).read()
    fns = cc.rb_gemm_functions(asm)
    assert len(fns) == 4
    for fn, ins in fns.items():
        reads, bad = cc.ahead_windows(ins)
        # 7 per 32-K step (gate/up: 4 steps per group; down: 4 + 2 for the 64-K tail)
        assert reads > 0 and reads % 7 == 0, (fn, reads)
        assert not bad, (fn, bad[:5])
    assert cc.check_rb_gemm(asm) == []  # what build.py runs before it links


def test_ahead_window_check_flags_a_touched_register():
    """The window check itself: a planted use of an in-flight destination, and
    a branch inside a window, are both reported."""
    ok = ["ds_read_b128 v[4:7], v2 offset:4096 ; ksl-ahead", "v_mfma_f32_16x16x32_f16 v[8:11], v[0:3], v[12:15], v[8:11]",
          "s_waitcnt lgkmcnt(0)", "v_mov_b32 v4, 0"]
    assert _ahead_windows(ok) == (1, [])
    touched = ["ds_read_b128 v[4:7], v2 offset:4096 ; ksl-ahead", "v_mov_b32 v30, v5", "s_waitcnt lgkmcnt(0)"]
    assert len(_ahead_windows(touched)[1]) == 1
    branch = ["ds_read_b128 v[4:7], v2 ; ksl-ahead", "s_cbranch_scc1 .LBB0_1", "s_waitcnt lgkmcnt(0)"]
    assert len(_ahead_windows(branch)[1]) == 1
