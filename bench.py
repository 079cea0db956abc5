#!/usr/bin/env python3
"""Benchmark: µs per RMSNorm + W4A16 MoE layer at a 256-token canvas, on one MI355X.

Workload layer_256: x bf16 [256, 2816] -> RMSNorm (w bf16 [2816], eps 1e-6) ->
W4A16 MoE (128 experts, top-8 from softmax of N(0,1) logits, renormalised;
gate/up [1408, 2816] group 128, down [2816, 704] group 64, asymmetric uint4,
fp16 scale/zero; SiLU-gated) -> fixed-order combine -> bf16 [256, 2816].
Synthetic seeded data. Inputs are resident in HBM before the timed region.

A "step" is one layer. Consecutive steps rotate over independent weight sets
(3 x 412 MB by default) so the 256 MB MALL cannot serve weights from cache.

Timed passes (all inside this process, same stream):
  1. value: K steps of the layer (one C call per step, four launches:
     routing + RMSNorm + fp16 activations, gate/up, down, combine), bracketed
     by synchronize; µs per layer = elapsed / K.
  2. per-kernel: K steps issued stage by stage with HIP events between the
     four launches; the average duration of each kernel, from which the
     dominant kernel's achieved bandwidth (roofline) is computed.
  3. cpu_baseline: the reference CPU path (torch eager, oracle/cpu_baseline.py)
     on the host cores, bounded to ~20 s.
Prints ONE JSON line on stdout; progress goes to stderr.
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


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--weight-sets", type=int, default=3)
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
    args = ap.parse_args()

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

    # ---- pass 1: whole-layer time -------------------------------------------
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

    # ---- pass 2: per-kernel durations with events between launches ----------
    kernels = {}
    if not args.skip_kernel_pass:
        stages = runner.stages(sets[0])
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)] for _ in range(args.steps)]
        for i in range(args.warmup):
            runner.run(xg, nwg, 1e-6, sets[i % len(sets)], idsg, wg)
        torch.cuda.synchronize()
        for i in range(args.steps):
            runner.run(xg, nwg, 1e-6, sets[i % len(sets)], idsg, wg, events=evs[i])
        torch.cuda.synchronize()
        for k, name in enumerate(stages):
            d = sorted(evs[i][k].elapsed_time(evs[i][k + 1]) * 1e3 for i in range(args.steps))
            kernels[name] = {"avg_us": sum(d) / len(d), "median_us": d[len(d) // 2]}
        tot = sum(v["avg_us"] for v in kernels.values())
        log("[bench] per-kernel avg us: " + ", ".join(f"{k} {v['avg_us']:.2f}" for k, v in kernels.items())
            + f" (sum {tot:.2f})")
        # parity of the staged output with the fused call on the same set
        step(sets[0])
        yf = y.clone()
        ys = runner.run(xg, nwg, 1e-6, sets[0], idsg, wg).clone()
        torch.cuda.synchronize()
        if not torch.equal(yf.view(torch.int16), ys.view(torch.int16)):
            log("[bench] WARNING: staged and fused outputs differ")

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

    gu_bytes = gateup_algorithmic_bytes(n_touched)
    roofline = None
    if kernels:
        gu_us = kernels["gateup"]["avg_us"] if "gateup" in kernels else kernels["ffn"]["avg_us"]
        ach = gu_bytes / (gu_us * 1e-6) / 1e9
        traffic = None
        tpath = os.path.join(ROOT, "profiles", "traffic_moe_gateup_layer256.json")
        if os.path.exists(tpath):
            with open(tpath) as f:
                traffic = json.load(f).get("hbm_bytes_per_launch")
        roofline = {"kernel": "gateup_act_kernel", "bound": "hbm", "achieved": round(ach, 1),
                    "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBPS, 4),
                    "traffic": traffic, "algorithmic_bytes": gu_bytes, "avg_us": round(gu_us, 3)}

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
            "layer_algorithmic_bytes": layer_bytes,
            "layer_GBps": round(layer_gbps, 1),
            "layer_frac_of_hbm_peak": round(layer_gbps / HBM_PEAK_GBPS, 4),
            "compute": "u4 weights, f16 MFMA operands, f32 accumulate, bf16 in/out",
            "parallelism": "single GPU",
            "kernels_us": {k: round(v["avg_us"], 3) for k, v in kernels.items()},
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
