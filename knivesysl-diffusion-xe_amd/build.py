"""Builds the gfx950 HIP library (libksl.so) in-tree with hipcc.

Usage: python knivesysl-diffusion-xe_amd/build.py   (or __graft_entry__.build()).
One shared object holds every kernel and the C ABI declared in include/ksl.h.
Each source compiles to its own object (in parallel), then one link.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libksl.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed-FP32 VALU ops are kept out of the device code on purpose
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]

# Per-source extra flags. moe_ffn.hip: the unit queue's atomic must stay one
# lane's atomic whose result is read cycles later; the atomic optimizer would
# rewrite it into a wave-wide scan that waits for the result at once.
EXTRA_FLAGS = {
    "moe_ffn.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *HIP_FLAGS, *EXTRA_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)} ({res.returncode}):\n{res.stderr[-8000:]}")
    return obj


def _check_generated_code(verbose: bool) -> None:
    """The row-block GEMMs' inline-asm LDS reads rely on the compiler leaving
    their destination registers alone until the wait that retires them: check
    that on this build's assembly (codegen_check.py) and refuse to link a
    library that breaks it."""
    import tempfile
    sys.path.insert(0, PKG_DIR)
    try:
        import codegen_check
    finally:
        sys.path.pop(0)
    src = os.path.join(CSRC, "moe_rbgemm.hip")
    with tempfile.TemporaryDirectory() as td:
        out = os.path.join(td, "moe_rbgemm.s")
        cmd = [HIPCC, *HIP_FLAGS, "-w", "--cuda-device-only", "-S", src, "-o", out]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc -S failed on moe_rbgemm.hip ({res.returncode}):\n{res.stderr[-8000:]}")
        errs = codegen_check.check_rb_gemm(open(out).read())
    if errs:
        raise RuntimeError("generated-code check failed (moe_rbgemm.hip):\n" + "\n".join(errs))


def build(verbose: bool = False) -> str:
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    os.makedirs(OBJ_DIR, exist_ok=True)
    workers = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", "8")), os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers + 1) as pool:
        check = pool.submit(_check_generated_code, verbose)
        objs = list(pool.map(lambda s: _compile(s, verbose), srcs))
        check.result()
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed ({res.returncode}):\n{res.stderr[-8000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    sys.exit(0)
