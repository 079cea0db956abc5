#!/usr/bin/env python3
"""Benchmark: µs per RMSNorm + W4A16 MoE layer at a 256-token canvas, on one MI355X.

Workload layer_256: x bf16 [256, 2816] -> RMSNorm (w bf16 [2816], eps 1e-6) ->
W4A16 MoE (128 experts, top-8 from softmax of N(0,1) logits, renormalised;
gate/up [1408, 2816] group 128, down [2816, 704] group 64, asymmetric uint4,
fp16 scale/zero; SiLU-gated) -> fixed-order combine -> bf16 [256, 2816].
Synthetic seeded data. Inputs are resident in HBM before the timed region.

A "step" is one layer. Consecutive steps rotate over independent weight sets
(3 x 412 MB by default) so the 256 MB MALL cannot serve weights from cache.

Settling: a fresh process's first ~20 ms of this workload run up to 20% slower
than its steady state (the per-step time decays over ~150 steps; 200 ms of
unrelated matmul or copy work beforehand does not remove it). Before the W
warmup steps of each timed pass the bench therefore runs the pass's own
workload for --settle-ms (50 ms by default; 0 turns it off), reported as
config.settle_ms; the warmup and timed steps are then as given.

Timed passes (all inside this process, on one stream):
  1. value: K steps of the layer (one C call per step: routing + RMSNorm +
     fp16 activations, gate/up, down, combine; with --ffn gate/up and down
     are one launch), bracketed by synchronize; µs per layer = elapsed / K.
  2. per-kernel: each stage's kernel alone, launches back to back between
     two HIP events on the same stream (the routing produced once; gate/up
     and down rotate over the weight sets), timed two ways: K launches from
     Python one by one (`eager_us`), and 20 launches captured in a HIP graph
     and replayed K/20 times, at least twice (`graph_us`). `avg_us` is the
     eager figure for gate/up and down, as the layer launches them, and the
     replay's for route_norm and combine, whose few microseconds of GPU work
     are paced by the host's launch cost when launched one by one from
     Python (a replay of back-to-back down launches reads ~3 us longer than
     the eager ones, so the expert GEMMs keep the eager figure). Achieved
     GB/s = the kernel's algorithmic bytes / that duration, and the dominant
     kernel's is the roofline. (Inside the layer,
     after route_norm, rocprofv3 reads the persistent gate/up kernel's
     dispatches ~4 us shorter than back to back; timing each stage inside the
     layer with events between the launches adds ~2-3 us of launch gap per
     stage instead, so the back-to-back figure stands.)
  3. RMSNorm alone at the rmsnorm_256 and rmsnorm_32k (+ qk-norm) shapes.
  4. cpu_baseline: the reference CPU path (torch eager, oracle/cpu_baseline.py)
     on every host core of the process's affinity set, bounded to ~20 s.
Prints ONE JSON line on stdout; progress goes to stderr.

HBM traffic per launch (roofline.traffic) comes from rocprofv3 counter runs
of this script, reduced by --summarize-pmc into profiles/traffic_layer256.json:
  rocprofv3 --pmc FETCH_SIZE --output-format csv -d <F> -- python3 bench.py --copy-calibration ...
  rocprofv3 --pmc WRITE_SIZE --output-format csv -d <W> -- python3 bench.py --copy-calibration ...
  python3 bench.py --summarize-pmc <F> <W>
FETCH_SIZE / WRITE_SIZE (KiB per dispatch) are scaled by what they read for
the copy of known size that --copy-calibration runs.
"""
from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
PKG = "knivesysl-diffusion-xe_amd"

METRIC = "µs per RMSNorm+W4A16 MoE layer at 256-tok canvas; achieved HBM GB/s (% peak)"
HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16/bf16 MFMA, MI355X

T, TOPK, E, H, I = 256, 8, 128, 2816, 704
GU_EXPERT_BYTES = 2 * I * (H // 2) + 2 * (2 * I * (H // 128) * 2)  # 1,982,464 + 123,904
DN_EXPERT_BYTES = H * (I // 2) + 2 * (H * (I // 64) * 2)           # 991,232 + 123,904


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def layer_algorithmic_bytes(n_experts_touched: int) -> int:
    """Compulsory HBM bytes of one layer: weights of every touched expert, the
    norm's input/weight/output, the MoE input and output, and the routing
    (ids int64 + weights fp32)."""
    w = n_experts_touched * (GU_EXPERT_BYTES + DN_EXPERT_BYTES)
    norm = T * H * 2 + H * 2 + T * H * 2
    moe_io = T * H * 2 + T * H * 2 + T * TOPK * (8 + 4)
    return w + norm + moe_io


def gateup_algorithmic_bytes(n_experts_touched: int) -> int:
    """Compulsory bytes of one gate/up launch: touched experts' gate/up weights,
    the fp16 activations read once, out2 written, sorted rows and offsets."""
    return (n_experts_touched * GU_EXPERT_BYTES + T * H * 2 + T * TOPK * I * 2 + T * TOPK * 4 + (E + 1) * 4)


def down_algorithmic_bytes(n_experts_touched: int) -> int:
    """Touched experts' down weights, out2 read once, out3 written, offsets."""
    return n_experts_touched * DN_EXPERT_BYTES + T * TOPK * I * 2 + T * TOPK * H * 2 + (E + 1) * 4


def route_norm_algorithmic_bytes() -> int:
    """x and the norm weight read, the fp16 activations written; ids read;
    sorted rows, inverse and offsets written."""
    return T * H * 2 + H * 2 + T * H * 2 + T * TOPK * 8 + 2 * T * TOPK * 4 + (E + 1) * 4


def combine_algorithmic_bytes() -> int:
    """out3 rows read once, the routing weights and inverse read, y written."""
    return T * TOPK * H * 2 + T * TOPK * (4 + 4) + T * H * 2


def stage_bytes(n_touched: int) -> dict:
    gu, dn = gateup_algorithmic_bytes(n_touched), down_algorithmic_bytes(n_touched)
    # the one-launch FFN: both weight sets; out2 is written and read back inside
    return {"route_norm": route_norm_algorithmic_bytes(), "gateup": gu, "down": dn,
            "ffn": gu + dn - T * TOPK * I * 2, "combine": combine_algorithmic_bytes()}


# rocprofv3 kernel names of the stages (substring match on the demangled name)
LATENCY_STAGES = ("route_norm", "combine")  # timed by graph replay (see pass 2)
STAGE_KERNELS = {"route_norm": "route", "gateup": "gateup_", "down": "down_kernel",
                 "ffn": "ffn_kernel", "combine": "combine_kernel"}


def summarize_pmc(fetch_dir: str, write_dir: str) -> int:
    """Per-kernel HBM bytes per dispatch from two rocprofv3 --pmc runs
    (FETCH_SIZE, WRITE_SIZE; KiB), each scaled by the factor that makes the
    --copy-calibration copies (512 MiB read + 512 MiB written each) read
    their known size; writes profiles/traffic_layer256.json."""
    import csv
    import glob

    def per_dispatch(d, counter):
        """{kernel name: {dispatch id: counter value summed over its rows}}"""
        vals: dict = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] == counter:
                    k = vals.setdefault(r["Kernel_Name"], {})
                    k[r["Dispatch_Id"]] = k.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
        return vals

    fd, wd = per_dispatch(fetch_dir, "FETCH_SIZE"), per_dispatch(write_dir, "WRITE_SIZE")
    fetch = {k: (sum(v.values()) / len(v), len(v)) for k, v in fd.items()}
    write = {k: (sum(v.values()) / len(v), len(v)) for k, v in wd.items()}
    copy_bytes = 512 << 20

    def copy_factor(table):
        # the largest single copy dispatch is one of the 512 MiB calibration copies
        vals = [x for k, v in table.items() if "copybuffer" in k.lower() for x in v.values()]
        return copy_bytes / (max(vals) * 1024.0) if vals and max(vals) > 0 else None

    fr, wr = copy_factor(fd), copy_factor(wd)
    out = {"source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over bench.py --copy-calibration",
           "unit": "bytes per dispatch", "fetch_scale": fr, "write_scale": wr, "kernels": {}}
    for stage, key in STAGE_KERNELS.items():
        names = [k for k in fetch if key in k]
        if not names:
            continue
        name = max(names, key=lambda k: fetch[k][1])
        f_kib, n = fetch[name]
        w_kib = write.get(name, (0.0, 0))[0]
        rd = f_kib * 1024.0 * (fr or 1.0)
        wt = w_kib * 1024.0 * (wr or 1.0)
        out["kernels"][stage] = {"kernel": name, "dispatches": n, "fetch_bytes": round(rd),
                                 "write_bytes": round(wt), "hbm_bytes_per_launch": round(rd + wt)}
    path = os.path.join(ROOT, "profiles", "traffic_layer256.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out, indent=1))
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--weight-sets", type=int, default=3)
    ap.add_argument("--settle-ms", type=float, default=50.0,
                    help="run each timed pass's workload this long before its warmup steps (0: off)")
    ap.add_argument("--act", choices=["silu", "gelu"], default="silu")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--skip-kernel-pass", action="store_true")
    ap.add_argument("--ffn", action="store_true",
                    help="pack the weights so gate/up and down run as one launch")
    ap.add_argument("--skip-prefill", action="store_true",
                    help="skip the prefill_8192 (Zipf routing) layer timing and its MFMA utilisation")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed region, copy a 512 MiB buffer 5 times (a kernel of known "
                         "traffic, the scale for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--skip-rmsnorm", action="store_true", help="skip the RMSNorm-alone timings")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="reduce two rocprofv3 --pmc output folders to profiles/traffic_layer256.json and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        return summarize_pmc(*args.summarize_pmc)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py measures one MI355X: this build runs the layer on a single GPU and has no "
            "multi-GPU path (see DESIGN.md for how the layer would shard). Run with --gpus 1.")
        return 2

    import torch
    pkg = importlib.import_module(PKG)
    wl = importlib.import_module(f"{PKG}.workloads")
    layer_mod = importlib.import_module(f"{PKG}.layer")
    lib = pkg._lib
    L = lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"[bench] device {torch.cuda.get_device_name(0)}; building inputs")

    x, nw, ids, w = wl.layer_inputs(T, 3)
    xg, nwg, idsg, wg = x.to(dev), nw.to(dev), ids.to(dev), w.to(dev)
    sets = []
    for s in range(args.weight_sets):
        exp = wl.make_experts(E, H, I, 100 + s, act=args.act, device=dev)
        sets.append(exp)
    n_touched = int(torch.unique(ids).numel())
    torch.cuda.synchronize()
    log(f"[bench] {args.weight_sets} weight sets x {sets[0].nbytes() / 1e6:.1f} MB; experts touched {n_touched}")

    runner = layer_mod.LayerRunner(T, TOPK, E, H, I, dev)
    ws = torch.empty(int(L.ksl_moe_workspace_bytes(T, TOPK, E, H, I)), dtype=torch.uint8, device=dev)
    y = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    p = lib.ptr
    st = lib.stream_of(xg)
    v2 = importlib.import_module(f"{PKG}.fused_moe_w4_v2")
    for exp in sets:
        v2._check_act(exp)
        v2._check_weights(exp, E, H, I)
        v2.enable_tiled_down(exp)  # load-time repack of the down weights (same results)
        if args.ffn:
            v2.enable_pack(exp)    # load-time pack for the one-launch expert FFN (same results)
    torch.cuda.synchronize()

    def step(exp):
        # one C call: routing + RMSNorm + fp16 activations, gate/up, down, combine
        rc = L.ksl_moe_layer_forward(p(xg), lib.DTYPE_BF16, H, p(nwg), lib.DTYPE_BF16, 1e-6,
                                     p(idsg), p(wg), lib.DTYPE_F32,
                                     p(exp.gu_q), p(exp.gu_s), p(exp.gu_z), p(exp.dn_q), p(exp.dn_s), p(exp.dn_z),
                                     lib.DN_LAYOUT_TILED, *v2.pack_ptrs(exp), T, TOPK, E, H, I, exp._ksl_act, p(y),
                                     lib.DTYPE_BF16, H,
                                     p(ws), ws.numel(), st)
        if rc:
            lib.check(rc, "ksl_moe_layer_forward")

    def settle(fn):
        # the workload itself, until settle_ms of GPU time have passed
        if args.settle_ms <= 0:
            return
        torch.cuda.synchronize()
        t_end = time.perf_counter() + args.settle_ms * 1e-3
        i = 0
        while time.perf_counter() < t_end:
            for _ in range(8):
                fn(sets[i % len(sets)])
                i += 1
            torch.cuda.synchronize()

    # ---- pass 1: whole-layer time -------------------------------------------
    settle(step)
    for i in range(args.warmup):
        step(sets[i % len(sets)])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for i in range(args.steps):
        step(sets[i % len(sets)])
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ev_ms = e0.elapsed_time(e1)
    ms_per_step = ev_ms / args.steps
    layer_us = ms_per_step * 1e3
    layer_bytes = layer_algorithmic_bytes(n_touched)
    layer_gbps = layer_bytes / (layer_us * 1e-6) / 1e9
    log(f"[bench] layer: {layer_us:.2f} us/step (events), wall {wall_ms / args.steps * 1e3:.2f} us/step; "
        f"{layer_gbps:.0f} GB/s = {100 * layer_gbps / HBM_PEAK_GBPS:.1f}% of 8 TB/s")

    # ---- pass 2: each stage's kernel alone, back to back ----------------------
    kernels = {}
    sbytes = stage_bytes(n_touched)
    if not args.skip_kernel_pass:
        stages = runner.stages(sets[0])
        runner.run(xg, nwg, 1e-6, sets[0], idsg, wg)  # routing, a16, out2, out3 for the launches below
        torch.cuda.synchronize()
        R = runner

        def launch(name, exp):
            if name == "route_norm":
                rc = L.ksl_moe_layer_route(p(idsg), T, TOPK, E, p(R.sorted_rows), p(R.offsets), p(R.inv), p(xg),
                                           lib.DTYPE_BF16, H, p(nwg), lib.DTYPE_BF16, 1e-6, H, p(R.a16),
                                           p(R.scratch), R.scratch.numel() * 4, st)
            elif name == "gateup":
                rc = L.ksl_moe_gateup_act(p(R.a16), p(R.sorted_rows), p(R.offsets), T, TOPK, p(exp.gu_q),
                                          p(exp.gu_s), p(exp.gu_z), E, H, I, exp._ksl_act, p(R.out2), st)
            elif name == "down":
                rc = L.ksl_moe_down(p(R.out2), p(R.offsets), p(exp.dn_q), p(exp.dn_s), p(exp.dn_z), E, H, I,
                                    T * TOPK, p(R.out3), v2.dn_layout(exp), st)
            elif name == "ffn":
                rc = L.ksl_moe_ffn(p(R.a16), p(R.sorted_rows), p(R.offsets), T, TOPK, p(exp.gu_pack),
                                   p(exp.dn_pack), E, H, I, exp._ksl_act, p(R.out2), p(R.out3), p(R.ctl), st)
            else:
                rc = L.ksl_moe_combine(p(R.out3), p(R.inv), p(wg), lib.DTYPE_F32, T, TOPK, H, p(R.y),
                                       lib.DTYPE_BF16, H, st)
            if rc:
                lib.check(rc, name)

        n_cap = 20
        for name in stages:
            for i in range(args.warmup):
                launch(name, sets[i % len(sets)])
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(args.steps):
                launch(name, sets[i % len(sets)])
            b.record()
            torch.cuda.synchronize()
            eager_us = a.elapsed_time(b) * 1e3 / args.steps
            # the same launches replayed from a graph: no host launch cost between
            # them (a few-microsecond kernel launched one by one from Python is
            # paced by the host); no memset nodes, every launch writes its outputs
            cap_stream = torch.cuda.Stream()
            cap_stream.wait_stream(torch.cuda.current_stream())
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=cap_stream):
                st = lib.stream_of(xg)  # the capturing stream
                for i in range(n_cap):
                    launch(name, sets[i % len(sets)])
            st = lib.stream_of(xg)
            torch.cuda.current_stream().wait_stream(cap_stream)
            graph.replay()
            torch.cuda.synchronize()
            reps = max(2, args.steps // n_cap)
            a.record()
            for _ in range(reps):
                graph.replay()
            b.record()
            torch.cuda.synchronize()
            graph_us = a.elapsed_time(b) * 1e3 / (reps * n_cap)
            del graph
            # the latency stages (a few microseconds each) are paced by the host's
            # launch cost when launched one by one: their figure is the replay's;
            # the expert GEMMs (tens of microseconds) keep the eager launches,
            # the way the layer launches them
            us = graph_us if name in LATENCY_STAGES else eager_us
            gbps = sbytes[name] / (us * 1e-6) / 1e9
            kernels[name] = {"avg_us": round(us, 3), "eager_us": round(eager_us, 3), "graph_us": round(graph_us, 3),
                             "algorithmic_bytes": sbytes[name], "GBps": round(gbps, 1),
                             "frac_of_hbm_peak": round(gbps / HBM_PEAK_GBPS, 4)}
        tot = sum(v["avg_us"] for v in kernels.values())
        log("[bench] per-kernel avg us (alone, back to back; eager launches / graph replay in brackets): "
            + ", ".join(f"{k} {v['avg_us']:.2f} [{v['eager_us']:.2f} / {v['graph_us']:.2f}] ({v['GBps']:.0f} GB/s)"
                        for k, v in kernels.items())
            + f" (sum {tot:.2f}, layer {layer_us:.2f})")
        # the staged launches give the fused call's bits
        step(sets[0])
        yf = y.clone()
        ys = runner.run(xg, nwg, 1e-6, sets[0], idsg, wg).clone()
        torch.cuda.synchronize()
        if not torch.equal(yf.view(torch.int16), ys.view(torch.int16)):
            log("[bench] WARNING: staged and fused outputs differ")

    # ---- pass 3: RMSNorm alone (rmsnorm_256, rmsnorm_32k + qk-norm) -----------
    rmsnorm = None
    if not args.skip_rmsnorm:
        def norm_us(xs, wt, n):
            rows, cols = xs[0].shape
            ys_ = [torch.empty_like(t) for t in xs]

            def one(i):
                rc = L.ksl_rmsnorm(p(xs[i % len(xs)]), lib.DTYPE_BF16, p(wt), lib.DTYPE_BF16, p(ys_[i % len(xs)]),
                                   lib.DTYPE_BF16, rows, cols, cols, cols, 1e-6, st)
                if rc:
                    lib.check(rc, "ksl_rmsnorm")

            for i in range(5):
                one(i)
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(n):
                one(i)
            b.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / n
            nbytes = 2 * rows * cols * 2 + cols * 2
            return us, nbytes / (us * 1e-6) / 1e9

        x0, w0, _ = wl.rmsnorm_256(0)
        u256, g256 = norm_us([x0.to(dev)], w0.to(dev), max(100, args.steps))
        x1, w1, qk, qkw, _ = wl.rmsnorm_32k(1)
        x1g = [x1.to(dev), x1.roll(1, 0).to(dev)]  # two inputs in turn: 2 x 184 MB, more than the MALL
        del x1
        u32k, g32k = norm_us(x1g, w1.to(dev), 50)
        del x1g
        uqk, gqk = norm_us([qk.to(dev)], qkw.to(dev), max(100, args.steps))
        rmsnorm = {"rmsnorm_256_us": round(u256, 3), "rmsnorm_256_GBps": round(g256, 1),
                   "rmsnorm_32k_us": round(u32k, 3), "rmsnorm_32k_GBps": round(g32k, 1),
                   "rmsnorm_32k_frac_of_hbm_peak": round(g32k / HBM_PEAK_GBPS, 4),
                   "qk_norm_4096x256_us": round(uqk, 3), "qk_norm_GBps": round(gqk, 1)}
        log(f"[bench] rmsnorm alone: [256, {H}] {u256:.2f} us ({g256:.0f} GB/s); [32768, {H}] {u32k:.2f} us "
            f"({g32k:.0f} GB/s = {100 * g32k / HBM_PEAK_GBPS:.1f}% of 8 TB/s); qk-norm [4096, 256] {uqk:.2f} us")
        torch.cuda.empty_cache()

    # ---- the router (the step before the layer; not part of `value`) --------
    router_us = None
    if not args.skip_kernel_pass:
        g = torch.Generator().manual_seed(7)
        r_scale = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
        r_proj = (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16).to(dev)
        r_pes = (1 + 0.1 * torch.randn(E, generator=g)).to(torch.bfloat16).to(dev)
        r_p = torch.empty(T, E, dtype=torch.float32, device=dev)
        r_w = torch.empty(T, TOPK, dtype=torch.float32, device=dev)
        r_ids = torch.empty(T, TOPK, dtype=torch.int64, device=dev)

        def route_step(stream):
            rc = L.ksl_moe_router(p(xg), lib.DTYPE_BF16, H, p(r_scale), p(r_proj), p(r_pes), lib.DTYPE_BF16, 1e-6,
                                  T, H, E, TOPK, p(r_p), p(r_w), p(r_ids), stream)
            if rc:
                lib.check(rc, "ksl_moe_router")

        for _ in range(args.warmup):
            route_step(st)
        torch.cuda.synchronize()
        ref_w, ref_ids = r_w.clone(), r_ids.clone()
        # a few microseconds of GPU work per call: launched one by one from Python
        # the host is the bottleneck, so the calls are captured in a graph and
        # replayed (no memset nodes: the router writes every output)
        n_cap = 20
        cap_stream = torch.cuda.Stream()
        cap_stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap_stream):
            cap = lib.stream_of(xg)  # the capturing stream
            for _ in range(n_cap):
                route_step(cap)
        torch.cuda.current_stream().wait_stream(cap_stream)
        graph.replay()
        torch.cuda.synchronize()
        if not (torch.equal(r_w, ref_w) and torch.equal(r_ids, ref_ids)):
            log("[bench] WARNING: router graph replay differs from the eager call")
        reps = max(1, args.steps // n_cap)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        router_us = e0.elapsed_time(e1) * 1e3 / (reps * n_cap)
        log(f"[bench] router (T={T}, E={E}, top-{TOPK}, not in the layer value): {router_us:.2f} us/call "
            f"(graph replay of {n_cap} calls)")

    # ---- the block's tail (the step after the layer; not part of `value`) ---
    # TF modeling_diffusion_gemma.py:733-743 after the experts: post norm 2,
    # + hidden_states_1, post norm, + residual, * layer_scalar. Fused: one
    # combine launch with the tail in its epilogue. Unfused, as the reference
    # runs it: the combine, then fused_rmsnorm, add, fused_rmsnorm, add, mul.
    tail = None
    if not args.skip_kernel_pass:
        frm = importlib.import_module(f"{PKG}.fused_rmsnorm")
        g = torch.Generator().manual_seed(8)
        t_h1 = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
        t_w2 = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
        t_wp = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
        t_ls = torch.tensor([0.75], dtype=torch.bfloat16, device=dev)
        t_y = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        t_m = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        b_y = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
        r_p = torch.empty(T, E, dtype=torch.float32, device=dev)
        b_w = torch.empty(T, TOPK, dtype=torch.float32, device=dev)
        b_ids = torch.empty(T, TOPK, dtype=torch.int64, device=dev)
        g = torch.Generator().manual_seed(7)
        r_scale = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
        r_proj = (0.05 * torch.randn(E, H, generator=g)).to(torch.bfloat16).to(dev)
        r_pes = (1 + 0.1 * torch.randn(E, generator=g)).to(torch.bfloat16).to(dev)
        exp0 = sets[0]
        unfused_out = []

        def tail_fused(stream):
            rc = L.ksl_moe_combine_post(p(runner.out3), p(runner.inv), p(wg), lib.DTYPE_F32, T, TOPK, H,
                                        p(t_h1), H, p(xg), H, p(t_w2), 1e-6, p(t_wp), 1e-6, p(t_ls), lib.DTYPE_BF16,
                                        p(t_y), H, stream)
            if rc:
                lib.check(rc, "ksl_moe_combine_post")

        def tail_unfused(stream):
            rc = L.ksl_moe_combine(p(runner.out3), p(runner.inv), p(wg), lib.DTYPE_F32, T, TOPK, H, p(t_m),
                                   lib.DTYPE_BF16, H, stream)
            if rc:
                lib.check(rc, "ksl_moe_combine")
            o = xg + frm.fused_rmsnorm(t_h1 + frm.fused_rmsnorm(t_m, t_w2, 1e-6), t_wp, 1e-6)
            o *= t_ls
            unfused_out.append(o)

        def block(stream):
            # the layer's whole MoE branch: router, then norm + experts + tail
            rc = L.ksl_moe_router(p(xg), lib.DTYPE_BF16, H, p(r_scale), p(r_proj), p(r_pes), lib.DTYPE_BF16, 1e-6,
                                  T, H, E, TOPK, p(r_p), p(b_w), p(b_ids), stream)
            if rc:
                lib.check(rc, "ksl_moe_router")
            rc = L.ksl_moe_block_forward(p(xg), H, p(nwg), 1e-6, p(b_ids), p(b_w), lib.DTYPE_F32,
                                         p(exp0.gu_q), p(exp0.gu_s), p(exp0.gu_z), p(exp0.dn_q), p(exp0.dn_s),
                                         p(exp0.dn_z), lib.DN_LAYOUT_TILED, *v2.pack_ptrs(exp0), T, TOPK, E, H, I,
                                         exp0._ksl_act, p(t_h1), H,
                                         p(t_w2), 1e-6,
                                         p(t_wp), 1e-6, p(t_ls), lib.DTYPE_BF16, p(b_y), H, p(ws), ws.numel(),
                                         stream)
            if rc:
                lib.check(rc, "ksl_moe_block_forward")

        def graph_us(fn, n_cap):
            for _ in range(3):
                fn(st)
            torch.cuda.synchronize()
            cap_stream = torch.cuda.Stream()
            cap_stream.wait_stream(torch.cuda.current_stream())
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=cap_stream):
                cap = lib.stream_of(xg)
                for _ in range(n_cap):
                    fn(cap)
            torch.cuda.current_stream().wait_stream(cap_stream)
            gr.replay()
            torch.cuda.synchronize()
            reps = max(1, args.steps // n_cap)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                gr.replay()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) * 1e3 / (reps * n_cap)

        fused_us = graph_us(tail_fused, 20)
        fused_y = t_y.clone()
        unfused_us = graph_us(tail_unfused, 20)
        ndiff = int((unfused_out[-1].view(torch.int16) != fused_y.view(torch.int16)).sum().item())
        block_us = graph_us(block, 5)
        tail = {"fused_us": round(fused_us, 3), "unfused_us": round(unfused_us, 3), "block_us": round(block_us, 3),
                "fused_vs_unfused_differing_elements": ndiff}
        log(f"[bench] block tail (not in the layer value): fused into the combine {fused_us:.2f} us, "
            f"combine + 5 separate calls {unfused_us:.2f} us ({ndiff} of {T * H} elements differ by the "
            f"row-sum order); router + block forward {block_us:.2f} us (graph replay)")

    # ---- the per-step sampler pass (not part of `value`) ---------------------
    # [256 canvas tokens, 262144 vocab] fp32 logits, 3 * N(0, 1) (the reference's
    # kill-test data): entropy alone, the Gumbel-max sample + argmax alone, and
    # the one-pass step (both from one read).
    sampler = None
    if not args.skip_kernel_pass:
        sops = importlib.import_module(f"{PKG}.fused_sampler_ops")
        V = 262144
        g = torch.Generator(device=dev)
        g.manual_seed(17)
        logits = 3.0 * torch.randn(T, V, generator=g, device=dev)
        nbytes = logits.numel() * 4

        def ev_us(fn, n):
            for _ in range(2):
                fn()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(n):
                fn()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) * 1e3 / n

        ent_us = ev_us(lambda: sops.fused_entropy(logits), 20)
        gum_us = ev_us(lambda: sops.gumbel_argmax_sample(logits, 1234), 10)
        step_us = ev_us(lambda: sops.sample_step(logits, 1234), 10)
        sampler = {"rows": T, "vocab": V, "logits_bytes": nbytes, "entropy_us": round(ent_us, 2),
                   "entropy_GBps": round(nbytes / (ent_us * 1e-6) / 1e9, 1),
                   "entropy_frac_of_hbm_peak": round(nbytes / (ent_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                   "gumbel_argmax_us": round(gum_us, 2), "sample_step_us": round(step_us, 2)}
        log(f"[bench] sampler [{T}, {V}] fp32: entropy {ent_us:.1f} us ({sampler['entropy_GBps']:.0f} GB/s), "
            f"gumbel+argmax {gum_us:.1f} us, one-pass step {step_us:.1f} us (the reference's two passes: "
            f"{ent_us + gum_us:.1f} us here)")
        del logits

    # ---- prefill_8192: T = 8192, Zipf(1.1) expert popularity (not part of `value`)
    # The same layer at prefill size, where the expert GEMMs are real
    # contractions: 2 * 65536 routed rows * (2I*H + H*I) = 779.5 GFLOP.
    prefill = None
    if not args.skip_kernel_pass and not args.skip_prefill:
        Tp = 8192
        xp_, nwp, idsp, wp = wl.layer_inputs(Tp, 4, zipf_s=1.1)
        xpg, nwpg, idspg, wpg = xp_.to(dev), nwp.to(dev), idsp.to(dev), wp.to(dev)
        yp = torch.empty(Tp, H, dtype=torch.bfloat16, device=dev)
        wsp = torch.empty(int(L.ksl_moe_workspace_bytes(Tp, TOPK, E, H, I)), dtype=torch.uint8, device=dev)
        flops = 2.0 * Tp * TOPK * (2 * I * H + H * I)
        counts = torch.bincount(idsp.reshape(-1), minlength=E)

        def pstep(exp):
            rc = L.ksl_moe_layer_forward(p(xpg), lib.DTYPE_BF16, H, p(nwpg), lib.DTYPE_BF16, 1e-6, p(idspg), p(wpg),
                                         lib.DTYPE_F32, p(exp.gu_q), p(exp.gu_s), p(exp.gu_z), p(exp.dn_q),
                                         p(exp.dn_s), p(exp.dn_z), lib.DN_LAYOUT_TILED, *v2.pack_ptrs(exp), Tp, TOPK, E, H, I,
                                         exp._ksl_act, p(yp), lib.DTYPE_BF16, H, p(wsp), wsp.numel(), st)
            if rc:
                lib.check(rc, "ksl_moe_layer_forward")

        settle(pstep)
        for i in range(3):
            pstep(sets[i % len(sets)])
        torch.cuda.synchronize()
        nrep = 10
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(nrep):
            pstep(sets[i % len(sets)])
        b.record()
        torch.cuda.synchronize()
        p_us = a.elapsed_time(b) * 1e3 / nrep
        prunner = layer_mod.LayerRunner(Tp, TOPK, E, H, I, dev)
        pstages = prunner.stages(sets[0])
        pev = [[torch.cuda.Event(enable_timing=True) for _ in range(len(pstages) + 1)] for _ in range(nrep)]
        for i in range(nrep):
            prunner.run(xpg, nwpg, 1e-6, sets[i % len(sets)], idspg, wpg, events=pev[i])
        torch.cuda.synchronize()
        pk = {name: sum(pev[i][k].elapsed_time(pev[i][k + 1]) for i in range(nrep)) * 1e3 / nrep
              for k, name in enumerate(pstages)}
        tflops = flops / (p_us * 1e-6) / 1e12
        gemm_us = pk["gateup"] + pk["down"]
        prefill = {"tokens": Tp, "zipf_s": 1.1, "max_rows_per_expert": int(counts.max()),
                   "min_rows_per_expert": int(counts.min()), "layer_us": round(p_us, 1),
                   "gflop": round(flops / 1e9, 1), "layer_TFLOPs": round(tflops, 1),
                   "mfma_utilisation": round(tflops / MFMA_PEAK_TFLOPS, 4),
                   "gemm_TFLOPs": round(flops / (gemm_us * 1e-6) / 1e12, 1),
                   "kernels_us": {k: round(v, 1) for k, v in pk.items()}}
        log(f"[bench] prefill_8192 (Zipf 1.1, rows/expert {int(counts.min())}..{int(counts.max())}): "
            f"{p_us:.1f} us/layer, {tflops:.1f} TFLOP/s = {100 * tflops / MFMA_PEAK_TFLOPS:.1f}% of the "
            f"2.5 PFLOP/s dense f16 MFMA peak; kernels " + ", ".join(f"{k} {v:.1f}" for k, v in pk.items()))
        del xpg, yp, wsp, prunner

    roofline = None
    if kernels:
        dom = max(kernels, key=lambda k: kernels[k]["avg_us"])
        kv = kernels[dom]
        traffic = traffic_kernel = None
        tpath = os.path.join(ROOT, "profiles", "traffic_layer256.json")
        if os.path.exists(tpath):
            with open(tpath) as f:
                t = json.load(f).get("kernels", {}).get(dom)
            if t:
                traffic, traffic_kernel = t["hbm_bytes_per_launch"], t["kernel"]
        roofline = {"kernel": dom, "bound": "hbm", "achieved": kv["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": kv["frac_of_hbm_peak"], "traffic": traffic, "traffic_kernel": traffic_kernel,
                    "algorithmic_bytes": kv["algorithmic_bytes"], "avg_us": kv["avg_us"]}

    if args.copy_calibration:
        nbytes = 512 << 20
        src = torch.ones(nbytes, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 5 copies of {nbytes} bytes")
        del src, dst

    # ---- pass 3: CPU baseline ------------------------------------------------
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline as cb
        log("[bench] cpu baseline (torch eager on host cores)...")
        expc = sets[0].to("cpu")
        act_code = 1 if args.act == "silu" else 0
        r = cb.time_layer(x, nw, 1e-6, expc, ids, w, act_code, budget_s=args.cpu_budget)
        cpu = {"value": round(r["dequant_per_call_s"] * 1e6, 1), "unit": "us", "cores": r["threads"],
               "kind": "port",
               "sample": (f"full layer_256 (all {E} experts), median of {r['dequant_per_call_runs']} runs "
                          f"after 1 warm-up, dequant per call; pre-dequantised weights: "
                          f"{r['predequant_s'] * 1e6:.0f} us (median of {r['predequant_runs']})"),
               "predequant_us": round(r["predequant_s"] * 1e6, 1)}
        log(f"[bench] cpu: {cpu['value']:.0f} us/layer dequant-per-call, {cpu['predequant_us']:.0f} us pre-dequantised, "
            f"{r['threads']} threads")

    out = {
        "metric": METRIC,
        "value": round(layer_us, 3),
        "unit": "us",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": (f"layer_256: RMSNorm bf16 [{T},{H}] + W4A16 MoE E={E} top-{TOPK} H={H} I={I} "
                         f"gu gs128 / dn gs64, {args.act}, fixed-order combine -> bf16"),
            "tokens": T, "experts": E, "topk": TOPK, "hidden": H, "intermediate": I,
            "act": args.act, "weight_sets": args.weight_sets, "experts_touched": n_touched,
            "settle_ms": args.settle_ms,
            "layer_algorithmic_bytes": layer_bytes,
            "layer_GBps": round(layer_gbps, 1),
            "layer_frac_of_hbm_peak": round(layer_gbps / HBM_PEAK_GBPS, 4),
            "compute": "u4 weights, f16 MFMA operands, f32 accumulate, bf16 in/out",
            "parallelism": "single GPU",
            "kernels": kernels,
            "rmsnorm_256_us": None if rmsnorm is None else rmsnorm["rmsnorm_256_us"],
            "rmsnorm_32k_us": None if rmsnorm is None else rmsnorm["rmsnorm_32k_us"],
            "rmsnorm": rmsnorm,
            "router_us": None if router_us is None else round(router_us, 3),
            "block_tail": tail,
            "sampler": sampler,
            "prefill_8192": prefill,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
