"""The generated code of the down kernel and of the persistent gate/up
kernel, checked on the CPU.

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
fragments, whose in-flight windows are checked below on the generated code.
The persistent gate/up kernel (one workgroup per CU walking several expert
column blocks, its consumers publishing row tables in LDS for its producer)
is run wave by wave the same way, with its item table and every wave's
barrier count checked."""
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


# ---- gate/up, flowing ring (gateup_flow_kernel): one persistent workgroup per CU
# The launch choice of csrc/moe_gemm.hip (gateup_flow_workgroups, GuFlowShape,
# launch_gateup_flow, gu_flow_paired_tile) restated for the emulated launches:
# NC = 11 consumer waves and one producer, ring depth 3, 176 columns per item.
GU_NC, GU_R, GU_MAXITEMS = 11, 3, 64


def _gu_flow_info_off(G):
    slot = 2 * GU_NC * 1024 + 4 * 2 * 1024  # weight blocks + two M tiles of activation blocks
    return GU_R * slot + 2 * (4 * 16 * GU_NC * G * 2) + 2 * 32 * 4


def _gu_flow_lds(G):
    return _gu_flow_info_off(G) + GU_MAXITEMS * 16


def _gu_flow_workgroups(items, H):
    W = CUS - CUS % 8
    G = H // 128
    if items <= CUS or items > W * GU_MAXITEMS or G < 8 or _gu_flow_lds(G) > 160 * 1024 - 64:
        return 0
    return W


def _gu_flow_pair(items, W, nb):
    return items == 2 * W and (W // 8) % nb == 0 and (items // 8) % nb == 0 and W // nb <= 64


def _gu_flow_tiles(w, W, items, nb, counts, pair):
    """Item tiles (expert * nb + column block) of workgroup w."""
    rm = (lambda b: (b % 8) * (items // 8) + b // 8) if items % 8 == 0 else (lambda b: b)
    tiles = [rm(w + k * W) for k in range(len(range(w, items, W)))]
    if pair:
        n = W // nb
        wj = [8 * nb * (j // 8) + j % 8 for j in range(n)]
        e1 = [rm(x) // nb for x in wj]
        e2 = [rm(x + W) // nb for x in wj]
        m1 = [int(counts[e]) for e in e1]
        m2 = [int(counts[e]) for e in e2]
        q = w // 8
        b, jm = q % nb, (q // nb) * 8 + w % 8
        r = sum(1 for j in range(n) if m1[j] > m1[jm] or (m1[j] == m1[jm] and e1[j] < e1[jm]))
        order2 = sorted(range(n), key=lambda j: (m2[j], e2[j]))
        tiles[1] = e2[order2[r]] * nb + b
    return tiles


def _sorted_rows(E, T, tk, kind, seed):
    rng = np.random.default_rng(seed)
    if kind == "uniform":
        ids = np.stack([rng.permutation(E)[:tk] for _ in range(T)])
    else:
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        p /= p.sum()
        ids = np.stack([rng.choice(E, tk, replace=False, p=p) for _ in range(T)])
    flat = ids.ravel()
    order = np.argsort(flat, kind="stable").astype(np.int64)
    return np.bincount(flat, minlength=E), order


GU_CASES = [
    # E, H, I, T, tk, routing, workgroups
    (128, 2816, 704, 256, 8, "uniform", (0, 77, 255)),   # the 256-token layer: balanced pairs
    (128, 2816, 704, 1024, 8, "zipf", (3, 200)),         # items of many passes, balanced pairs
    (128, 2816, 704, 16, 2, "uniform", (0, 1, 130)),     # mostly empty items
    (256, 1024, 704, 128, 8, "uniform", (0, 255)),       # G = 8, the shortest passes; four items each (no pairs)
    (256, 3072, 352, 128, 8, "uniform", (5, 254)),       # G = 24, the largest LDS, balanced pairs
    (192, 2816, 704, 256, 8, "uniform", (0, 100, 255)),  # three items per workgroup
]


@pytest.mark.parametrize("E,H,I,T,tk,routing,wgs", GU_CASES)
def test_gateup_flow_kernel_addresses_and_register_flow(down_asm, E, H, I, T, tk, routing, wgs):
    """Every wave of a few workgroups of gateup_flow_kernel (SiLU): the
    consumers (wave 0 fills the item table, with the balanced second items,
    and each pass's successor token ids in LDS) and then the producer, whose
    direct global->LDS loads are addressed from those tables; all accesses in
    bounds, no poisoned address or operand, LDS within the launch's dynamic
    size, the item table as restated here (every item owned by exactly one
    workgroup), and the same number of barriers in every wave."""
    G = H // 128
    nb = I // 176
    items = E * nb
    W = _gu_flow_workgroups(items, H)
    assert W == 256, "the flowing kernel runs for this shape"
    pair = _gu_flow_pair(items, W, nb)
    fn = "_ZN3ksl12_GLOBAL__N_118gateup_flow_kernelILi1ELi11EEEvNS0_6GuArgsEiii"
    ins, labels = emu.load_kernel(down_asm, fn)
    counts, order = _sorted_rows(E, T, tk, routing, E + H + I + T)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    nrows = T * tk
    lds = _gu_flow_lds(G)
    all_tiles = sorted(t for w in range(W) for t in _gu_flow_tiles(w, W, items, nb, counts, pair))
    assert all_tiles == list(range(items))
    bufs, base = {}, 0x7F0000000000

    def alloc(name, size):
        nonlocal base
        bufs[name] = (base, base + size)
        base += ((size + 0xFFFFF) // 0x100000 + 16) * 0x100000
        return bufs[name][0]

    p_a16 = alloc("a16", T * H * 2)
    p_rows = alloc("sorted_rows", nrows * 4)
    p_off = alloc("offsets", (E + 1) * 4)
    p_q = alloc("gu_q", E * 2 * I * H // 2)
    p_s = alloc("gu_s", E * 2 * I * G * 2)
    p_z = alloc("gu_z", E * 2 * I * G * 2)
    p_out2 = alloc("out2", nrows * I * 2)
    p_karg = alloc("kernarg", 128)
    early = 1 if nrows >= E else 0
    karg = struct.pack("<QQQQQQQiiiiiii", p_a16, p_rows, p_off, p_q, p_s, p_z, p_out2, tk, I, H, early, W, items,
                       int(pair))
    assert len(karg) == 84
    karg += b"\0" * 4
    mem = {p_karg + k: struct.unpack("<I", karg[k:k + 4])[0] for k in range(0, len(karg), 4)}
    mem.update({p_off + 4 * e: int(offsets[e]) for e in range(E + 1)})
    mem.update({p_rows + 4 * r: int(order[r]) for r in range(nrows)})
    info_off = _gu_flow_info_off(G)

    def lds_i32(lds_map, addr):
        v = 0
        for k in range(4):
            byte, known = lds_map.get(addr + k, (0, False))
            assert known, ("unknown LDS byte", addr + k)
            v |= int(byte) << (8 * k)
        return v - (1 << 32) if v & 0x80000000 else v

    checked = 0
    for wg in wgs:
        assert wg < W
        tiles = _gu_flow_tiles(wg, W, items, nb, counts, pair)
        shared = None
        barriers = []
        for wave_id in range(GU_NC + 1):  # consumers first: they fill the tables the producer reads
            w = emu.Wave(mem, p_karg, wg, wave_id, bufs, lds)
            if shared is not None:
                w.lds = shared
            emu.run(ins, labels, w, max_steps=20_000_000)
            shared = w.lds
            checked += w.accesses
            barriers.append(w.barriers)
            assert not w.errors, (wg, wave_id, w.errors[:4])
            if wave_id == 0:
                for k, t in enumerate(tiles):
                    e = t // nb
                    got = [lds_i32(shared, info_off + 16 * k + 4 * f) for f in range(4)]
                    assert got == [int(offsets[e]), int(counts[e]), e, (t % nb) * 176], (wg, k, got)
        # every wave takes the same barriers: the first, one more when the first
        # item has no rows (and a later one has), one per group of each pass
        npass = sum(-(-int(counts[t // nb]) // 32) for t in tiles)
        late = 1 if counts[tiles[0] // nb] == 0 and npass > 0 else 0
        assert barriers == [1 + late + npass * G] * (GU_NC + 1), (wg, barriers, npass)
    assert checked > 0
