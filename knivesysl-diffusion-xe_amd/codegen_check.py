"""Checks on the generated gfx950 assembly that the compiler cannot make itself.

The row-block GEMMs (csrc/moe_rbgemm.hip) read the next M tile's activation
fragment from LDS by inline asm (`ds_read_b128 ...; ksl-ahead`) and wait for
it just before use: the compiler believes the four destination registers
written at the asm statement, so nothing it emits between the read and the
`s_waitcnt lgkmcnt(0)` that retires it may read or write them, and no branch
may fall inside that window. build.py runs this check on every build and
fails the build on a violation; tests/test_cpu_codegen.py runs it too.
"""
from __future__ import annotations

import re


def vregs(tok: str) -> set[int]:
    """VGPR numbers named by one assembly operand (v7, v[4:7])."""
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def ahead_windows(lines: list[str]) -> tuple[int, list]:
    """For every `ds_read_b128 ...; ksl-ahead`, the instructions up to the next
    s_waitcnt that retires it. Returns (reads, violations): a violation is an
    instruction in the window that reads or writes one of the destination
    registers, or a branch or label inside the window."""
    reads, bad = 0, []
    for i, line in enumerate(lines):
        if "ksl-ahead" not in line or "ds_read_b128" not in line:
            continue
        reads += 1
        dst = vregs(line.split()[1].rstrip(","))
        if len(dst) != 4:
            bad.append((i, "destination is not four registers: " + line))
            continue
        for j in range(i + 1, len(lines)):
            s = lines[j].split(";")[0].strip()
            if not s:
                continue
            if s.startswith("s_waitcnt") and "lgkmcnt(0)" in s:
                break
            if s.endswith(":") or s.startswith("s_cbranch") or s.startswith("s_branch") or s.startswith("s_setpc"):
                bad.append((i, s))
                break
            used = set()
            for t in s.split()[1:]:
                used |= vregs(t.strip(","))
            if used & dst:
                bad.append((i, s))
        else:
            bad.append((i, "no wait before the function ends"))
    return reads, bad


def rb_gemm_functions(asm_text: str) -> dict[str, list[str]]:
    """The instruction lines of every rb_gemm_kernel instance in an assembly file."""
    text = asm_text.split("\n")
    out = {}
    for i0, l in enumerate(text):
        if l.startswith("_ZN3ksl12_GLOBAL__N_114rb_gemm_kernel") and l.split(";")[0].strip().endswith(":"):
            fn = l.split(":")[0]
            ins = []
            for l2 in text[i0 + 1:]:
                if l2.startswith(".Lfunc_end"):
                    break
                ins.append(l2.strip())
            out[fn] = ins
    return out


def check_rb_gemm(asm_text: str) -> list[str]:
    """Violations of the ahead-read windows over every rb_gemm_kernel instance
    (7 reads per 32-K step: gate/up 4 steps per 128-K group, down 4 + 2 for
    its 64-K tail, times however many copies of the loop body the compiler
    emits), as messages; empty when the code is sound."""
    errs = []
    fns = rb_gemm_functions(asm_text)
    if len(fns) != 4:
        errs.append(f"expected 4 rb_gemm_kernel instances, found {len(fns)}")
    for fn, ins in fns.items():
        reads, bad = ahead_windows(ins)
        if reads == 0 or reads % 7:
            errs.append(f"{fn}: {reads} ahead reads (expected a positive multiple of 7)")
        for b in bad[:5]:
            errs.append(f"{fn}: in-flight register or branch in an ahead-read window: {b}")
    return errs
