#!/usr/bin/env python3
"""W4A8 per-group linear throughput at QwQ-32B shapes on one MI355X.

Metric: "W4A8 GEMM TOPS + weight GB/s (% roofline), QwQ-32B
shapes, M=1..4096".

One step = the decode configuration: dynamic per-token int8
quant + W4A8 GEMM for each QwQ-32B projection (qkv 5120->7168, o 5120->5120,
gate_up 5120->55296, down 27648->5120) at M in {1, 4, 16, 64}, group 128 --
16 linears.  Cold protocol (the reference's, int4_cube_lab/host/mg_harness.h:42,
:215-219): every projection has a pool of >= 8 distinct weight copies totalling
>= 1 GiB; each of the 16 linears of a step reads its own copy, and per-shape
timings rotate through the pool, so no weight byte is re-read within 1 GiB of
traffic -- far beyond the 256 MB Infinity Cache.  Each step is replayed as a
HIP graph (8 graphs over distinct copies).

``value`` = algorithmic bytes of the 16 linears per step / step time, in
GB/s: GEMM bytes N*K/2 + (K/G)*N*2 + M*K + 4*M + 2*M*N (weights, group scales, int8
activations, token scales, bf16 output)
plus quant bytes 2*M*K + M*K + 2*M.  Inputs are resident in HBM before the
timed region.  Per-shape kernel times (graph replays of back-to-back
launches between HIP events), prefill TOPS and a CPU baseline
(the reference's own C++ CPU GEMM on configs[0], timed on this host) are
reported in the same JSON line.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, TOP/s
GROUP = 128
DECODE_MS = (1, 4, 16, 64)
PROJS = ("qkv_proj", "o_proj", "gate_up_proj", "down_proj")


def gemm_bytes(M, N, K, G=GROUP):
    return N * K // 2 + (K // G) * N * 2 + M * K + 4 * M + 2 * M * N


def quant_bytes(M, K):
    return 2 * M * K + M * K + 2 * M


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cold-bytes", type=float, default=1.0, help="GiB of distinct weight copies to rotate")
    ap.add_argument("--detail-launches", type=int, default=40)
    ap.add_argument("--prefill-m", default="1024,4096,16384")
    ap.add_argument("--no-decoder", action="store_true",
                    help="skip configs[4]: the 64-layer QwQ-32B-shaped decoder, 1024-token prompts + "
                         "--decoder-steps greedy decode steps at concurrency 1, 8, 64 (run by default)")
    ap.add_argument("--decoder-layers", type=int, default=64)
    ap.add_argument("--decoder-steps", type=int, default=256,
                    help="greedy decode steps per concurrency (configs[4] states 256)")
    ap.add_argument("--no-compat", action="store_true",
                    help="skip the reference-compat mid-group pair (group 1024, asymmetric) at M 1/16/64/1024/4096")
    ap.add_argument("--no-config4", action="store_true",
                    help="skip configs[3]: groups 64/256/512 at M 16/4096, gate_up with the fused SwiGLU")
    ap.add_argument("--no-tp4", action="store_true",
                    help="skip the tensor-parallel shard shapes (TP=4 slices of the four projections)")
    ap.add_argument("--no-perchannel", action="store_true",
                    help="skip the per-channel (group = K) points beside the reference's published ones")
    ap.add_argument("--no-attention", action="store_true",
                    help="skip the decoder's attention kernel (w4a8_attention) at concurrency 1/8/64")
    ap.add_argument("--attention-sweep", action="store_true",
                    help="with the attention leg: also every split size (chunks per split 1-20) per concurrency")
    ap.add_argument("--no-detail", action="store_true", help="only the timed steps (for profiling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: each decode linear once (eager) on cold weights, then a "
                         "256 MiB device copy of known size for calibrating the byte counters")
    ap.add_argument("--trace-summary", metavar="DB",
                    help="summarize a rocprofv3 --kernel-trace database (rocpd SQLite) as markdown and exit")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                    help="turn two rocprofv3 --pmc databases of a --pmc-probe run (FETCH_SIZE, WRITE_SIZE) into "
                         "the per-shape HBM traffic table (markdown on stdout) and exit")
    ap.add_argument("--pmc-json", metavar="OUT",
                    help="with --pmc-summary or --prefill-pmc-summary: also write the traffic figures as JSON")
    ap.add_argument("--prefill-probe", type=int, metavar="M", default=0,
                    help="for rocprofv3 runs: each configs[2] projection's prefill GEMM at M rows three times "
                         "(eager, group 128), then a 256 MiB device copy of known size")
    ap.add_argument("--decoder-probe", type=int, metavar="B", default=0,
                    help="for rocprofv3 runs: the --decoder-layers decoder at concurrency B, a 1024-token prefill "
                         "(cache of 1024 + 256 positions, as the decoder leg), then its captured decode step "
                         "replayed 5 + 10 times (the 10 between two marker launches are the ones "
                         "--decoder-trace-summary reads)")
    ap.add_argument("--decoder-trace-summary", metavar="DB",
                    help="summarize a --kernel-trace database of a --decoder-probe run: kernels per decode step "
                         "and their time, as markdown, and exit")
    ap.add_argument("--decode-pmc-summary", nargs="+", metavar="DB",
                    help="summarize rocprofv3 databases of a --pmc-probe run (counter passes, then a "
                         "--kernel-trace database last) for the 16 decode GEMM calls as markdown and exit")
    ap.add_argument("--prefill-pmc-summary", nargs="+", metavar="DB",
                    help="summarize rocprofv3 databases of a --prefill-probe run (counter passes, then a "
                         "--kernel-trace database last) for the prefill GEMM kernels as markdown and exit")
    args = ap.parse_args()
    if args.trace_summary:
        trace_summary(args.trace_summary)
        return
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary, args.pmc_json)
        return
    if args.prefill_pmc_summary:
        prefill_pmc_summary(args.prefill_pmc_summary, args.pmc_json)
        return
    if args.decode_pmc_summary:
        decode_pmc_summary(args.decode_pmc_summary)
        return
    if args.decoder_trace_summary:
        decoder_trace_summary(args.decoder_trace_summary)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the W4A8 linear is "
              f"a per-GPU kernel (tensor-parallel shards run the same kernel on their slice)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import __graft_entry__ as ge
    pkg = ge.package()
    synth = pkg.synth
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    props = torch.cuda.get_device_properties(dev)

    if args.prefill_probe:
        prefill_probe(pkg, dev, args.prefill_probe)
        return
    if args.decoder_probe:
        decoder_probe(pkg, dev, args.decoder_layers, args.decoder_probe)
        return

    # ---------------------------------------------------------------- data
    gen = torch.Generator(device=dev)

    def make_pool(p, G, codes_dist, scale_dtype, seed, shape=None):
        """>= 8 distinct repacked copies of projection p's weight (or of a [N, K] = shape
        slice), >= cold_bytes in total."""
        K, N = shape if shape is not None else synth.QWQ_SHAPES[p]
        per = gemm_bytes(0, N, K, G)
        n = max(8, math.ceil(args.cold_bytes * 2 ** 30 / per))
        pool = []
        for r in range(n):
            gen.manual_seed(seed + r)
            if codes_dist == "uniform":
                codes = torch.randint(-8, 8, (N, K), dtype=torch.int8, device=dev, generator=gen)
            else:   # round(clip(N(0, 2.5), -8, 7)), configs[3]
                codes = torch.randn((N, K), device=dev, generator=gen).mul_(2.5).clamp_(-8, 7).round_().to(torch.int8)
            w_q = pkg.packing.pack_int4(codes)
            del codes
            ws = (torch.rand((K // G, N), device=dev, generator=gen) * 0.018 + 0.002).to(scale_dtype)
            pool.append(torch.ops.npu.w4a8_repack(w_q, ws, K, G))
            del w_q, ws
        return pool

    weights = {p: make_pool(p, GROUP, "uniform", torch.float16, 1000 * pi) for pi, p in enumerate(PROJS)}
    pool_bytes = {p: len(weights[p]) * gemm_bytes(0, synth.QWQ_SHAPES[p][1], synth.QWQ_SHAPES[p][0])
                  for p in PROJS}
    log(f"bench: {props.name}, weight pools " +
        ", ".join(f"{p} {len(weights[p])} x {pool_bytes[p] / len(weights[p]) / 1e6:.1f} MB" for p in PROJS))
    xs = {}
    for M in DECODE_MS:
        for p in PROJS:
            K, _ = synth.QWQ_SHAPES[p]
            xb = synth.activations(M, K, seed=10 * M + PROJS.index(p))
            xs[(M, p)] = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
    torch.cuda.synchronize()

    n_graphs = 8

    def step(r):
        # linear (M index mi, projection p) of graph r reads copy 4r + mi of p's pool
        outs = []
        for mi, M in enumerate(DECODE_MS):
            for p in PROJS:
                K, N = synth.QWQ_SHAPES[p]
                wt, st = weights[p][(len(DECODE_MS) * r + mi) % len(weights[p])]
                # quant + GEMM (one fused launch where w4a8_linear qualifies)
                outs.append(torch.ops.npu.w4a8_linear(xs[(M, p)], wt, st, N, K, GROUP))
        return outs

    if args.pmc_probe:
        for i, M in enumerate(DECODE_MS):
            for j, p in enumerate(PROJS):
                K, N = synth.QWQ_SHAPES[p]
                wt, st = weights[p][i % len(weights[p])]
                a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(xs[(M, p)])
                torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP)
        src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log("bench: pmc probe done (16 decode linears, then one 268435456-byte device copy)")
        return

    # ---------------------------------------------------------------- graphs
    cap = torch.cuda.Stream(device=dev)
    cap.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(cap):
        for r in range(n_graphs):    # warm the capture stream (any allocation happens here, not in capture)
            step(r)
    torch.cuda.current_stream(dev).wait_stream(cap)
    torch.cuda.synchronize()
    graphs = []
    for r in range(n_graphs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            step(r)
        graphs.append(g)
    torch.cuda.synchronize()

    bytes_per_step = sum(gemm_bytes(M, synth.QWQ_SHAPES[p][1], synth.QWQ_SHAPES[p][0]) +
                         quant_bytes(M, synth.QWQ_SHAPES[p][0]) for M in DECODE_MS for p in PROJS)

    # ---------------------------------------------------------------- timed region
    for i in range(args.warmup):
        graphs[i % n_graphs].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        graphs[(args.warmup + i) % n_graphs].replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    clocks = gpu_clocks()   # right after the timed region (the clocks ramp down when idle)
    value = bytes_per_step / (ms_per_step * 1e-3) / 1e9
    log(f"bench: {ms_per_step:.4f} ms/step, {value:.1f} GB/s over {bytes_per_step / 1e6:.1f} MB/step")

    result = {
        "metric": "W4A8 GEMM TOPS + weight GB/s (% roofline), QwQ-32B shapes, M=1..4096",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded): bf16 N(0,1) activations with 0.1% outlier channels x20; int4 codes "
                "uniform [-8,7]; fp16 group scales U[0.002,0.02]",
        "config": {"workload": "configs[1]: decode W4A8 linears (quant+GEMM), QwQ-32B qkv/o/gate_up/down, "
                               "M in {1,4,16,64}, group 128, cold (every linear reads its own weight copy; "
                               "per-projection pools of " +
                               ", ".join(f"{len(weights[p])}" for p in PROJS) +
                               f" copies, {sum(pool_bytes.values()) / 2 ** 30:.2f} GiB)",
                   "group": GROUP, "linears_per_step": len(DECODE_MS) * len(PROJS),
                   "bytes_per_step": bytes_per_step},
    }
    if args.no_detail:
        print(json.dumps(result), flush=True)
        return

    # ---------------------------------------------------------------- per-shape kernel times
    T = args.detail_launches
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    # Per-shape timings run on their own stream (warm-up launches and graph
    # replays alike), so a kernel trace of this command separates them from
    # the step graphs by stream; `--trace-summary` reports per stream.
    shape_stream = torch.cuda.Stream(device=dev)

    def time_graph(fn, reps=3, stream=None):
        st = stream if stream is not None else shape_stream
        with torch.cuda.stream(st):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            fn()
        torch.cuda.synchronize()
        times = []
        with torch.cuda.stream(st):
            g.replay()
            for _ in range(reps):
                e0, e1 = ev(), ev()
                e0.record(st)
                g.replay()
                e1.record(st)
                e1.synchronize()
                times.append(e0.elapsed_time(e1) * 1e3)   # us
        torch.cuda.synchronize()
        del g
        return sorted(times)[len(times) // 2]

    shapes = []
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    floors = {}
    reads = {}
    copy_dst = {}
    tot_bytes = tot_us = 0.0
    for M in DECODE_MS:
        for p in PROJS:
            K, N = synth.QWQ_SHAPES[p]
            a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(xs[(M, p)])

            def gemms(a_q=a_q, a_s=a_s, p=p, K=K, N=N):
                for i in range(T):
                    wt, st = weights[p][i % len(weights[p])]
                    torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP)

            def quants(M=M, p=p):
                for _ in range(T):
                    torch.ops.npu.w4a8_quant_pertoken(xs[(M, p)])

            def linears(M=M, p=p, K=K, N=N):
                for i in range(T):
                    wt, st = weights[p][i % len(weights[p])]
                    torch.ops.npu.w4a8_linear(xs[(M, p)], wt, st, N, K, GROUP)

            if p not in copy_dst:
                copy_dst[p] = torch.empty_like(weights[p][0][0])

            def floor_reads(p=p):
                # the same pool rotation moved by a stock torch device copy (weight tiles)
                for i in range(T):
                    copy_dst[p].copy_(weights[p][i % len(weights[p])][0])

            def floor_read(p=p):
                # the same pool rotation streamed by the library's read-floor kernel
                # (w4a8_read_floor): the time the weight tiles take to read, nothing else
                lib = pkg._abi.lib()
                st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
                for i in range(T):
                    wt = weights[p][i % len(weights[p])][0]
                    pkg._abi.check(lib.w4a8_read_floor(wt.data_ptr(), wt.numel(), sink.data_ptr(), st),
                                   "w4a8_read_floor")

            us = time_graph(gemms) / T
            qus = time_graph(quants) / T
            fus = time_graph(floor_reads) / T if M == DECODE_MS[0] else floors[p]
            floors[p] = fus
            rus = time_graph(floor_read) / T if M == DECODE_MS[0] else reads[p]
            reads[p] = rus
            # quant + GEMM through w4a8_linear, on the step's stream
            lus = time_graph(linears, stream=torch.cuda.current_stream(dev)) / T
            x0 = xs[(M, p)]
            fused = bool(pkg._abi.lib().w4a8_linear_fused(x0.data_ptr(), x0.stride(0), M, N, K, GROUP))
            b = gemm_bytes(M, N, K)
            tot_bytes += b
            tot_us += us
            shapes.append({"proj": p, "M": M, "N": N, "K": K, "gemm_us": round(us, 3),
                           "gemm_GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                           "TOPS": round(2 * M * N * K / us / 1e6, 2), "quant_us": round(qus, 3),
                           "linear_us": round(lus, 3), "linear_fused": fused,
                           "copy_us": round(fus, 3), "read_floor_us": round(rus, 3),
                           "vs_read_floor": round(rus / us, 4)})
            cgb = 2 * weights[p][0][0].numel() / fus / 1e3
            log(f"  {p:13s} M={M:3d}: gemm {us:8.2f} us {b / us / 1e3:7.1f} GB/s ({b / us / 1e3 / HBM_PEAK_GBS:.1%})"
                f"  quant {qus:6.2f} us  linear {lus:7.2f} us{' (fused)' if fused else ''}  "
                f"copy {fus:6.2f} us ({cgb:6.0f} GB/s)  read floor {rus:6.2f} us ({rus / us:.0%} of gemm time)")
    achieved = tot_bytes / tot_us / 1e3
    # HBM bytes per launch from the two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) recorded in
    # profiles/ (the command is in the summary), each scaled by a 256 MiB copy's reading.
    traffic, traffic_src = None, ROOT / "profiles" / "gemm_decode_kernel_traffic.json"
    if traffic_src.exists():
        traffic = round(json.loads(traffic_src.read_text())["avg_traffic_bytes"])
    result["roofline"] = {
        "kernel": ("decode W4A8 GEMM per call: gemm_decode_kernel; gemm_wide_kernel for gate_up at M=16 and 64 "
                   "and down at M=16 (K split over 12 workgroups), gemm_prefill_cols_kernel's 64-row tile for down at M=64 (K split "
                   "over 6 workgroups), each split call followed by wide_reduce_kernel -- all 16 configs[1] "
                   "shapes, cold"),
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
        "per_launch_bytes_avg": round(tot_bytes / len(shapes)), "launch_us_avg": round(tot_us / len(shapes), 3),
        "timing": "HIP events around graph replays of back-to-back launches on the launch stream",
        "traffic_source": str(traffic_src.relative_to(ROOT)) if traffic is not None else None,
    }
    result["decode_shapes"] = shapes
    result["stock_copy"] = {
        "what": ("per projection, a stock torch device copy (Tensor.copy_) of each pool copy's repacked weight "
                 "tiles into one buffer of the same size, graph-replayed back to back over the same rotation as "
                 "the GEMMs: what stock code moves at each weight size, cold reads plus writes"),
        "us": {p: round(floors[p], 3) for p in PROJS},
        "GBs_read_plus_write": {p: round(2 * weights[p][0][0].numel() / floors[p] / 1e3, 1) for p in PROJS}}
    result["read_floor"] = {
        "what": ("per projection, the library's streaming-read kernel (w4a8_read_floor: 256-thread workgroups, "
                 "two 16-byte non-temporal loads per thread) over each pool copy's repacked weight tiles, "
                 "graph-replayed back to back over the same rotation as the GEMMs: the time the weight bytes "
                 "alone take to read cold; decode_shapes[*].vs_read_floor = read_floor_us / gemm_us"),
        "us": {p: round(reads[p], 3) for p in PROJS},
        "GBs": {p: round(weights[p][0][0].numel() / reads[p] / 1e3, 1) for p in PROJS},
        "hbm_frac": {p: round(weights[p][0][0].numel() / reads[p] / 1e3 / HBM_PEAK_GBS, 4) for p in PROJS}}
    result["gpu_clocks"] = {"after_timed_region": clocks,
                            "note": "rocm-smi reading; the peaks above are MI355X's published figures (2.4 GHz)"}

    # ---------------------------------------------------------------- prefill
    prefill = []
    for M in [int(m) for m in args.prefill_m.split(",") if m]:
        for p in PROJS:
            K, N = synth.QWQ_SHAPES[p]
            x = synth.activations_device(M, K, seed=M, device=dev)
            # the first quant call on these freshly allocated buffers, then the warm kernel time
            torch.cuda.synchronize()
            e0, e1 = ev(), ev()
            e0.record()
            a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x)
            e1.record()
            torch.cuda.synchronize()
            q_first = e0.elapsed_time(e1) * 1e3
            Tq = max(2, min(20, int(4e4 // max(1, M))))

            def quants_p(x=x, Tq=Tq):
                for _ in range(Tq):
                    torch.ops.npu.w4a8_quant_pertoken(x)

            q_us = time_graph(quants_p) / Tq
            Tp = max(2, min(10, int(2e4 // max(1, M))))

            def gemms(a_q=a_q, a_s=a_s, p=p, K=K, N=N, Tp=Tp):
                for i in range(Tp):
                    wt, st = weights[p][i % len(weights[p])]
                    torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP)

            us = time_graph(gemms) / Tp
            tops = 2 * M * N * K / us / 1e6
            prefill.append({"proj": p, "M": M, "gemm_us": round(us, 2), "TOPS": round(tops, 1),
                            "mfma_frac": round(tops / INT8_PEAK_TOPS, 4),
                            "GBs": round(gemm_bytes(M, N, K) / us / 1e3, 1),
                            "quant_us": round(q_us, 2), "quant_GBs": round(quant_bytes(M, K) / q_us / 1e3, 1),
                            "quant_first_call_us": round(q_first, 1)})
            log(f"  prefill {p:13s} M={M:5d}: {us:9.1f} us {tops:7.1f} TOPS ({tops / INT8_PEAK_TOPS:.1%} of int8 peak)"
                f"  quant {q_us:8.1f} us ({quant_bytes(M, K) / q_us / 1e3:6.0f} GB/s; first call {q_first:8.1f} us)")
            del x, a_q, a_s
    result["prefill_shapes"] = prefill
    if prefill:
        # right after the MFMA-bound prefill loop: the clock that kernel ran at
        result["gpu_clocks"]["after_prefill"] = gpu_clocks()
        at = [r for r in prefill if r["M"] == 4096] or prefill
        ops = sum(2 * r["M"] * synth.QWQ_SHAPES[r["proj"]][1] * synth.QWQ_SHAPES[r["proj"]][0] for r in at)
        us_tot = sum(r["gemm_us"] for r in at)
        ach = ops / us_tot / 1e6
        result["roofline_prefill"] = {
            "kernel": f"gemm_prefill_cols_kernel (128 x 32 wave tiles), the four configs[2] projections at "
                      f"M={at[0]['M']}, group 128 "
                      f"(algorithmic ops 2*M*N*K per call over the summed call times)",
            "bound": "mfma", "achieved": round(ach, 1), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
            "frac": round(ach / INT8_PEAK_TOPS, 4), "traffic": None,
            "per_launch_ops_avg": round(ops / len(at)), "launch_us_avg": round(us_tot / len(at), 2),
            "timing": "HIP events around graph replays of back-to-back launches"}
        # HBM bytes per launch from the committed counter passes of the same
        # kernel and M (FETCH_SIZE + WRITE_SIZE, scaled by a 256 MiB copy)
        tsrc = ROOT / "profiles" / "gemm_prefill_cols_kernel_traffic.json"
        if tsrc.exists():
            tj = json.loads(tsrc.read_text())
            if tj.get("M") == at[0]["M"]:
                result["roofline_prefill"].update(
                    traffic=round(tj["avg_traffic_bytes"]), alg_bytes_avg=round(tj["avg_alg_bytes"]),
                    traffic_source=str(tsrc.relative_to(ROOT)))

        # the vendor library's plain int8 GEMM on the same shapes and M (no group
        # scales, no fold, no unpack; int8 weights, int32 output): what the
        # matrix cores give a library kernel under the same sustained load
        result["int8_library_ref"] = int8_library_ref(dev, synth, at[0]["M"], time_graph, prefill)

    # the decode pools are not needed past this point
    weights = None
    torch.cuda.empty_cache()
    # ---------------------------------------------------------------- per-channel (group = K)
    if not args.no_perchannel:
        result["perchannel_shapes"] = perchannel(pkg, dev, synth, make_pool, time_graph, T)
    # ---------------------------------------------------------------- mid-group variants
    if not args.no_config4:
        result["config4_shapes"] = config4(pkg, dev, synth, make_pool, time_graph, T)
    if not args.no_compat:
        result["compat_shapes"] = compat(pkg, dev, synth, time_graph, T, args.cold_bytes)
    # ---------------------------------------------------------------- TP=4 shard shapes (one GPU's slice)
    if not args.no_tp4:
        result["tp4_shapes"] = tp4(pkg, dev, synth, make_pool, time_graph, T)
    # ---------------------------------------------------------------- decoder attention
    if not args.no_attention:
        result["attention_shapes"] = attention_bench(pkg, dev, time_graph, args.cold_bytes, args.attention_sweep)
    # ---------------------------------------------------------------- decoder forward
    if not args.no_decoder:
        result["decoder"] = decoder_bench(pkg, dev, args.decoder_layers, steps=args.decoder_steps, attention="torch")
        result["decoder_attention_kernel"] = decoder_bench(pkg, dev, args.decoder_layers, steps=args.decoder_steps,
                                                           attention="hip")

    # ---------------------------------------------------------------- CPU baseline
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(pkg, dev, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def config4(pkg, dev, synth, make_pool, time_graph, T):
    """the four projections at M in {16, 4096} with groups 64/256/512, bf16 scales and
    clipped-normal codes; gate_up followed by SwiGLU (output 27648), fused and unfused."""
    import numpy as np
    import torch
    rows = []
    for G in (64, 256, 512):
        for pi, p in enumerate(PROJS):
            K, N = synth.QWQ_SHAPES[p]
            pool = make_pool(p, G, "clipped_normal", torch.bfloat16, 50000 + 1000 * pi + G)
            for M in (16, 4096):
                x = torch.from_numpy(synth.activations(M, K, seed=M + G).view(np.int16)).view(torch.bfloat16).to(dev)
                a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, G)
                n = T if M <= 64 else 4
                ops = {"gemm": lambda wt, st: torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, G)}
                if p == "gate_up_proj":
                    I = N // 2

                    def unfused(wt, st):
                        y = torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, G)
                        return torch.nn.functional.silu(y[:, :I]) * y[:, I:]

                    ops = {"swiglu_fused": lambda wt, st: torch.ops.npu.w4a8_gemm_swiglu(a_q, a_s, wt, st, N, K, G),
                           "swiglu_unfused": unfused}
                for name, op in ops.items():
                    def launches(op=op):
                        for i in range(n):
                            op(*pool[i % len(pool)])
                    us = time_graph(launches) / n
                    # the fused op writes [M, N/2] instead of [M, N]
                    b = gemm_bytes(M, N, K, G) - (M * N if name == "swiglu_fused" else 0)
                    tops = 2 * M * N * K / us / 1e6
                    rows.append({"proj": p, "M": M, "group": G, "op": name, "us": round(us, 2),
                                 "GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                                 "TOPS": round(tops, 1), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4)})
                    log(f"  config4 {p:13s} G={G:3d} M={M:5d} {name:15s}: {us:9.2f} us "
                        f"{b / us / 1e3:7.1f} GB/s ({b / us / 1e3 / HBM_PEAK_GBS:.1%})  {tops:7.1f} TOPS "
                        f"({tops / INT8_PEAK_TOPS:.1%})")
                del x, a_q, a_s
            del pool
            torch.cuda.empty_cache()
    return rows


def decoder_probe(pkg, dev, layers, B, prompt=1024, steps=256, warm=5, timed=10):
    """configs[4]'s decode step for a kernel trace, on the cache the bench's decoder leg uses
    (`prompt` + `steps` positions): a prefill of `prompt` tokens, the step captured once, `warm`
    graph replays, then `timed` replays between two marker launches (a tiny weight repack, a
    kernel the decode step never runs) that --decoder-trace-summary cuts at."""
    import torch
    cfg = pkg.decoder.DecoderConfig(layers=layers)
    m = pkg.decoder.W4A8Decoder(cfg, batch=B, max_len=prompt + steps, device=dev, seed=7)
    tokens = torch.randint(0, cfg.vocab, (B, prompt), generator=torch.Generator().manual_seed(0)).to(dev)
    first = m.prefill(tokens)
    torch.cuda.synchronize()
    g = m.capture()
    m.tokens.copy_(first)
    m.pos.fill_(prompt)
    w_q = torch.zeros((16, 64), dtype=torch.int8, device=dev)
    w_s = torch.ones((1, 16), dtype=torch.float16, device=dev)
    torch.cuda.synchronize()
    for _ in range(warm):
        g.replay()
    torch.ops.npu.w4a8_repack(w_q, w_s, 128, 128)      # marker
    for _ in range(timed):
        g.replay()
    torch.ops.npu.w4a8_repack(w_q, w_s, 128, 128)      # marker
    torch.cuda.synchronize()
    log(f"bench: decoder probe done ({layers} layers, concurrency {B}, {timed} timed decode-step replays)")


def decoder_trace_summary(db, timed=10):
    """Kernels of one decode step (the average over the replays between the two markers of a
    --decoder-probe run) as markdown."""
    import collections
    import sqlite3
    rows = sqlite3.connect(db).execute("select name, duration, start, end from kernels order by start").fetchall()
    marks = [i for i, r in enumerate(rows) if "repack_weight_kernel" in r[0]]
    if len(marks) < 2:
        raise SystemExit("bench.py: no --decoder-probe markers in this trace")
    tail = [r for r in rows[marks[-2] + 1:marks[-1]] if "repack_scale_kernel" not in r[0]]
    agg = collections.defaultdict(lambda: [0, 0.0])
    for name, d, _, _ in tail:
        k = name.replace("(anonymous namespace)", "~").split("(")[0].strip()
        if k.startswith("void "):
            k = k[5:]
        agg[k[:96]][0] += 1
        agg[k[:96]][1] += d / 1e3
    busy = sum(v[1] for v in agg.values()) / timed
    span = (tail[-1][3] - tail[0][2]) / 1e3 / timed
    print(f"Decode step, kernel trace of {timed} graph replays: {len(tail) / timed:.0f} launches per step, "
          f"{busy:.0f} us of kernel time per step, {span:.0f} us from the first kernel's start to the last "
          f"kernel's end per step (rocprof's timestamps; a traced run is slower than an untraced one).\n")
    print("| kernel | per step | calls per step | us per call |\n|---|---:|---:|---:|")
    for k, (c, t) in sorted(agg.items(), key=lambda kv: -kv[1][1])[:24]:
        print(f"| `{k}` | {t / timed:.1f} us | {c / timed:.0f} | {t / c:.2f} |")


def attention_bench(pkg, dev, time_graph, cold_gib, sweep=False, batches=(1, 8, 64)):
    """The decoder's attention kernel at QwQ-32B heads (40 query heads, 8 KV heads, head_dim
    128) over the bench decoder's cache (1024 + 256 positions).  Decode: one query token per
    sequence at position 1100 (a split launch and, with more than one split, the combine),
    cold -- each launch reads its own copy of the cache from a pool of >= cold_gib GiB --
    against the attended K and V bytes B * 8 * 1101 * 128 * 2 * 2; beside it
    scaled_dot_product_attention (efficient backend) on the same cache in [L, D] layout.
    Prefill: a 1024-token prompt per sequence (causal), against the MFMA work
    4 * B * 40 * 128 * S (S + 1) / 2 flops and the 2.5 PFLOP/s bf16 peak."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel
    H, KVH, D, L, P = 40, 8, 128, 1280, 1100
    G = H // KVH
    rows = []
    for B in batches:
        per = B * KVH * L * D * 2 * 2
        n = max(4, min(256, math.ceil(cold_gib * 2 ** 30 / per)))
        kp = torch.randn((n, B, KVH, L, D), device=dev).to(torch.bfloat16)
        vp = torch.randn((n, B, KVH, D, L), device=dev).to(torch.bfloat16)
        q = torch.randn((B, 1, H, D), device=dev).to(torch.bfloat16)
        pos = torch.full((1,), P, dtype=torch.int64, device=dev)
        base = pkg.ops.attention_chunks_per_split(B, H, KVH, L)
        attended = B * KVH * (P + 1) * D * 2 * 2

        def run(cps):
            for i in range(n):
                torch.ops.npu.w4a8_attention(q, kp[i], vp[i], pos, L, cps, True)
        row = {"phase": "decode", "concurrency": B, "position": P, "cache": L, "chunks_per_split": base,
               "splits": -(-(L // 64) // base)}
        us = time_graph(lambda: run(base)) / n
        row.update({"us": round(us, 2), "attended_MB": round(attended / 1e6, 2),
                    "TB_s": round(attended / us / 1e6, 3), "frac_8TBs": round(attended / us / 1e6 / 8.0, 3)})
        if sweep:
            row["sweep_us"] = {c: round(time_graph(lambda c=c: run(c)) / n, 2) for c in range(1, 21)}
        # scaled_dot_product_attention over the same positions ([L, D] values, a bf16 mask)
        ks, vs = kp[: min(n, 8)], vp[: min(n, 8)].transpose(3, 4).contiguous()
        mask = torch.where(torch.arange(L, device=dev) > P, float("-inf"), 0.0).to(torch.bfloat16)
        qg = q.view(B, KVH, G, D)

        def sd():
            with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
                for i in range(ks.shape[0]):
                    torch.nn.functional.scaled_dot_product_attention(qg, ks[i], vs[i],
                                                                     attn_mask=mask.expand(B, KVH, G, L))
        row["sdpa_us"] = round(time_graph(sd) / ks.shape[0], 2)
        rows.append(row)
        log(f"  attention decode B={B:3d}: {us:7.2f} us ({row['TB_s']:.2f} TB/s of attended K/V, "
            f"{row['splits']} splits), sdpa {row['sdpa_us']:.2f} us")
        del kp, vp, ks, vs
        torch.cuda.empty_cache()
    for B, S in ((1, 1024), (8, 1024), (64, 1024)):
        k = torch.randn((B, KVH, L, D), device=dev).to(torch.bfloat16)
        vt = torch.randn((B, KVH, D, L), device=dev).to(torch.bfloat16)
        q = torch.randn((B, S, H, D), device=dev).to(torch.bfloat16)
        pos = torch.zeros((1,), dtype=torch.int64, device=dev)
        cps = pkg.ops.attention_chunks_per_split(B, H, KVH, L)
        us = time_graph(lambda: torch.ops.npu.w4a8_attention(q, k, vt, pos, L, cps, False))
        flops = 4 * B * H * D * S * (S + 1) / 2
        row = {"phase": "prefill", "concurrency": B, "prompt": S, "us": round(us, 1),
               "us_per_sequence": round(us / B, 1), "TFLOP_s": round(flops / us / 1e6, 1),
               "frac_bf16_peak": round(flops / us / 1e6 / 2500.0, 3)}
        if B == 1:
            qs = q.view(B, S, KVH, G, D).permute(0, 2, 3, 1, 4).reshape(B, KVH, G * S, D).contiguous()
            kk, vv = k[:, :, :S].contiguous(), vt[..., :S].transpose(2, 3).contiguous()
            pmask = torch.full((S, S), float("-inf"), device=dev).triu_(1).repeat(G, 1).to(torch.bfloat16)

            def sdp():
                with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
                    torch.nn.functional.scaled_dot_product_attention(
                        qs, kk, vv, attn_mask=pmask.view(1, 1, G * S, S).expand(B, KVH, G * S, S))
            row["sdpa_us"] = round(time_graph(sdp), 1)
        rows.append(row)
        log(f"  attention prefill B={B:3d} S={S}: {us:9.1f} us ({row['TFLOP_s']:.0f} TFLOP/s causal)"
            + (f", sdpa {row['sdpa_us']:.1f} us" if "sdpa_us" in row else ""))
        del k, vt, q
        torch.cuda.empty_cache()
    return rows


def decoder_bench(pkg, dev, layers, prompt=1024, steps=256, batches=(1, 8, 64), attention="torch"):
    """prefill tokens/s and greedy decode tokens/s of the QwQ-32B-shaped decoder
    (random W4A8 weights at group 128, decode steps replayed from a HIP graph).  attention
    "torch" is the config as stated -- bf16 attention left on PyTorch-ROCm (batched products
    below decoder.SDPA_MIN_BATCH sequences, scaled_dot_product_attention from it on); "hip"
    runs the same model on this build's attention kernel (w4a8_attention, the decode step
    with the rotary embedding and the KV append fused in)."""
    import torch
    cfg = pkg.decoder.DecoderConfig(layers=layers)
    t0 = time.perf_counter()
    m = pkg.decoder.W4A8Decoder(cfg, batch=batches[0], max_len=prompt + steps, device=dev, seed=7,
                                attention=attention)
    torch.cuda.synchronize()
    log(f"  decoder: {layers} layers built in {time.perf_counter() - t0:.1f} s")
    # one untimed short prefill first: the first call loads the torch/BLAS code paths
    m.resize(batches[0], prompt + steps)
    m.prefill(torch.randint(0, cfg.vocab, (batches[0], 64), device=dev))
    torch.cuda.synchronize()
    rows = []
    for B in batches:
        m.resize(B, prompt + steps)
        toks = torch.randint(0, cfg.vocab, (B, prompt), device=dev, generator=torch.Generator(device=dev).manual_seed(B))
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        torch.cuda.synchronize()
        e[0].record()
        first = m.prefill(toks)
        e[1].record()
        m.capture()
        torch.cuda.synchronize()
        e[2].record()
        out = m.decode(first, prompt, steps, graph=True)
        e[3].record()
        torch.cuda.synchronize()
        pre_ms, dec_ms = e[0].elapsed_time(e[1]), e[2].elapsed_time(e[3])
        rows.append({"concurrency": B, "prompt_tokens": prompt, "decode_steps": steps,
                     "prefill_ms": round(pre_ms, 1), "prefill_tok_s": round(B * prompt / pre_ms * 1e3, 1),
                     "decode_ms_per_step": round(dec_ms / steps, 3), "decode_tok_s": round(B * steps / dec_ms * 1e3, 1),
                     "attention": {"hip": "w4a8_attention", "sdpa": "scaled_dot_product_attention",
                                   "matmul": "batched products"}[m.attention],
                     "last_tokens": [int(t) for t in out[-1][:4].tolist()]})
        log(f"  decoder ({m.attention}) B={B:3d}: prefill {pre_ms:9.1f} ms ({B * prompt / pre_ms * 1e3:9.0f} tok/s), decode "
            f"{dec_ms / steps:7.3f} ms/step ({B * steps / dec_ms * 1e3:8.1f} tok/s)")
    del m
    torch.cuda.empty_cache()
    return rows


# The reference's published per-channel W4A8 kernel times on its 910B4
# (int4_cube_lab/results/midgroup_w4a8_qwen.csv, rows "w4a8_pc": avg_us per
# projection and M; the CSV line of each value in the key).
REF_PERCHANNEL_US = {
    ("qkv_proj", 1): (28.26, 3), ("qkv_proj", 4): (28.46, 6), ("qkv_proj", 16): (28.57, 9),
    ("qkv_proj", 64): (34.81, 12), ("qkv_proj", 1024): (186.51, 21),
    ("o_proj", 1): (23.98, 24), ("o_proj", 4): (24.10, 27), ("o_proj", 16): (24.32, 30),
    ("o_proj", 64): (28.97, 33), ("o_proj", 1024): (136.85, 42),
    ("gate_up_proj", 1): (132.83, 45), ("gate_up_proj", 4): (132.80, 48), ("gate_up_proj", 16): (132.91, 51),
    ("gate_up_proj", 64): (165.74, 54), ("gate_up_proj", 1024): (1564.72, 63),
    ("down_proj", 1): (72.17, 66), ("down_proj", 4): (72.35, 69), ("down_proj", 16): (72.78, 72),
    ("down_proj", 64): (97.98, 75), ("down_proj", 1024): (710.03, 84),
}


def perchannel(pkg, dev, synth, make_pool, time_graph, T, ms=(1, 4, 16, 64, 1024)):
    """Per-channel weights (one group spanning K): GEMM time per projection and M on cold
    pools, beside the reference's published time for the same point."""
    import numpy as np
    import torch
    rows = []
    for pi, p in enumerate(PROJS):
        K, N = synth.QWQ_SHAPES[p]
        pool = make_pool(p, K, "uniform", torch.bfloat16, 5000 + 100 * pi)
        for M in ms:
            x = torch.from_numpy(synth.activations(M, K, seed=M + 50).view(np.int16)).view(torch.bfloat16).to(dev)
            a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, K)
            Tm = T if M <= 64 else max(2, T // 8)

            def gemms(a_q=a_q, a_s=a_s, K=K, N=N, Tm=Tm):
                for i in range(Tm):
                    wt, st = pool[i % len(pool)]
                    torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, K)

            us = time_graph(gemms) / Tm
            b = gemm_bytes(M, N, K, K)
            ref_us, line = REF_PERCHANNEL_US[(p, M)]
            rows.append({"proj": p, "M": M, "N": N, "K": K, "group": K, "gemm_us": round(us, 3),
                         "GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                         "TOPS": round(2 * M * N * K / us / 1e6, 1),
                         "reference_910b4_us": ref_us,
                         "reference_source": f"int4_cube_lab/results/midgroup_w4a8_qwen.csv:{line}",
                         "speedup_vs_reference": round(ref_us / us, 2)})
            log(f"  per-channel {p:13s} M={M:5d}: {us:9.2f} us {b / us / 1e3:7.1f} GB/s "
                f"({b / us / 1e3 / HBM_PEAK_GBS:.1%}), reference 910B4 {ref_us} us")
        del pool
        torch.cuda.empty_cache()
    return rows


# The reference's published mid-group W4A8 kernel times on its 910B4 (group 1024,
# asymmetric weights, per-(token, group) activation scales: the compat pair's
# arithmetic), int4_cube_lab/results/midgroup_w4a8_qwen.csv rows "w4a8_mg_asym".
REF_MIDGROUP_US = {
    ("qkv_proj", 1): (31.12, 4), ("qkv_proj", 16): (31.07, 10), ("qkv_proj", 64): (40.65, 13),
    ("qkv_proj", 1024): (274.92, 22),
    ("o_proj", 1): (26.33, 25), ("o_proj", 16): (26.27, 31), ("o_proj", 64): (32.67, 34),
    ("o_proj", 1024): (197.95, 43),
    ("gate_up_proj", 1): (148.48, 46), ("gate_up_proj", 16): (148.41, 52), ("gate_up_proj", 64): (206.43, 55),
    ("gate_up_proj", 1024): (2225.47, 64),
    ("down_proj", 1): (76.23, 67), ("down_proj", 16): (76.13, 73), ("down_proj", 64): (108.13, 76),
    ("down_proj", 1024): (1012.92, 85),
}


# Tensor-parallel shards at TP=4 of QwQ-32B's projections (one GPU's slice;
# the reference's open question about its kernel at per-rank shapes,
# MGCKPT/P7_LOWDIM_KERNEL.md:13-21): column-parallel qkv/gate_up split N,
# row-parallel o/down split K.  (K, N) per projection.
TP4_SHAPES = {"qkv_proj": (5120, 1792), "o_proj": (1280, 5120), "gate_up_proj": (5120, 13824),
              "down_proj": (6912, 5120)}


def tp4(pkg, dev, synth, make_pool, time_graph, T, ms=(1, 16, 64, 1024)):
    """One GPU's TP=4 slice of every projection, group 128, cold pools, through w4a8_linear
    (quant + GEMM) and the GEMM alone."""
    import numpy as np
    import torch
    rows = []
    for pi, p in enumerate(PROJS):
        K, N = TP4_SHAPES[p]
        pool = make_pool(p, GROUP, "uniform", torch.float16, 90000 + 100 * pi, shape=(K, N))
        for M in ms:
            x = torch.from_numpy(synth.activations(M, K, seed=M + 70).view(np.int16)).view(torch.bfloat16).to(dev)
            a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x)
            Tm = T if M <= 64 else max(2, T // 8)

            def gemms(a_q=a_q, a_s=a_s, K=K, N=N, Tm=Tm):
                for i in range(Tm):
                    wt, st = pool[i % len(pool)]
                    torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP)

            def linears(x=x, K=K, N=N, Tm=Tm):
                for i in range(Tm):
                    wt, st = pool[i % len(pool)]
                    torch.ops.npu.w4a8_linear(x, wt, st, N, K, GROUP)

            us, lus = time_graph(gemms) / Tm, time_graph(linears) / Tm
            b = gemm_bytes(M, N, K)
            tops = 2 * M * N * K / us / 1e6
            rows.append({"proj": p, "shard": "N/4" if p in ("qkv_proj", "gate_up_proj") else "K/4", "M": M,
                         "N": N, "K": K, "gemm_us": round(us, 3), "linear_us": round(lus, 3),
                         "GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                         "TOPS": round(tops, 1), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4)})
            log(f"  tp4 {p:13s} N={N:5d} K={K:5d} M={M:5d}: gemm {us:9.2f} us {b / us / 1e3:7.1f} GB/s "
                f"({b / us / 1e3 / HBM_PEAK_GBS:.1%}) {tops:7.1f} TOPS  linear {lus:9.2f} us")
            del x, a_q, a_s
        del pool
        torch.cuda.empty_cache()
    return rows


def compat(pkg, dev, synth, time_graph, T, cold_bytes):
    """The reference-compat pair (midgroup_quant_a + midgroup_w4a8_gemm, group 1024, asymmetric) on
    the reference's packed tensors, cold pools as for the main path."""
    import numpy as np
    import torch
    G = 1024
    gen = torch.Generator(device=dev)
    rows = []
    for pi, p in enumerate(PROJS):
        K, N = synth.QWQ_SHAPES[p]
        kb, ng = pkg.geometry.kpad(K, G) // 2, pkg.geometry.num_groups(K, G)
        per = N * kb + ng * N * 8
        pool = []
        for r in range(max(8, math.ceil(cold_bytes * 2 ** 30 / per))):
            gen.manual_seed(70000 + 1000 * pi + r)
            w_q = torch.randint(-128, 128, (N, kb), dtype=torch.int8, device=dev, generator=gen)
            ws = (torch.rand((ng, N), device=dev, generator=gen) * 0.018 + 0.002).to(torch.bfloat16)
            wz = torch.randint(-8, 8, (ng, N), device=dev, generator=gen).to(torch.bfloat16)
            wk = torch.zeros((ng, N), dtype=torch.int32, device=dev)
            pool.append((w_q, ws, wk, wz))
        tiles = [torch.ops.npu.midgroup_tile_weights(w[0], K, G) for w in pool]
        for M in (1, 16, 64, 1024, 4096):
            x = torch.from_numpy(synth.activations(M, K, seed=M).view(np.int16)).view(torch.bfloat16).to(dev)
            a = torch.ops.npu.midgroup_quant_a(x, G)
            n = T if M <= 64 else 4

            def gemms(a=a, K=K, n=n):
                for i in range(n):
                    torch.ops.npu.midgroup_w4a8_gemm(*a, *pool[i % len(pool)], K, G)

            def quants(x=x, n=n):
                for _ in range(n):
                    torch.ops.npu.midgroup_quant_a(x, G)

            def gemms_rows(a=a, K=K, n=n, M=M):
                for i in range(n):
                    torch.ops.npu.midgroup_w4a8_gemm(*a, *pool[i % len(pool)], K, G, M)

            def gemms_tiled(a=a, K=K, N=N, n=n, M=M):
                for i in range(n):
                    w_q, ws, wk, wz = pool[i % len(pool)]
                    torch.ops.npu.midgroup_w4a8_gemm_tiled(*a, tiles[i % len(pool)], ws, wk, wz, N, K, G, M)

            us, qus = time_graph(gemms) / n, time_graph(quants) / n
            Mp = a[0].shape[0]
            # the real rows only (midgroup_linear / the vLLM method), where quant_a padded them
            rus = time_graph(gemms_rows) / n if Mp > M else us
            # the weight as 1 KB tiles made once at load (the vLLM method's and MidGroupW4A8Linear's layout)
            tus = time_graph(gemms_tiled) / n
            b = N * kb + ng * N * 6 + Mp * kb * 2 + ng * Mp * 6 + 2 * Mp * N
            tops = 2 * M * N * K / us / 1e6
            row = {"proj": p, "M": M, "gemm_us": round(us, 2), "GBs": round(b / us / 1e3, 1),
                   "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "TOPS": round(tops, 1),
                   "mfma_frac": round(tops / INT8_PEAK_TOPS, 4), "quant_a_us": round(qus, 2),
                   "gemm_real_rows_us": round(rus, 2), "gemm_tiled_rows_us": round(tus, 2)}
            if (p, M) in REF_MIDGROUP_US:
                ref_us, line = REF_MIDGROUP_US[(p, M)]
                row.update(reference_910b4_us=ref_us,
                           reference_source=f"int4_cube_lab/results/midgroup_w4a8_qwen.csv:{line}",
                           speedup_vs_reference=round(ref_us / us, 2))
            rows.append(row)
            log(f"  compat {p:13s} M={M:5d}: gemm {us:9.2f} us {b / us / 1e3:7.1f} GB/s "
                f"({b / us / 1e3 / HBM_PEAK_GBS:.1%}) {tops:7.1f} TOPS  quant_a {qus:7.2f} us"
                f"  real rows {rus:9.2f} us  tiled {tus:9.2f} us")
            del x, a
        del pool, tiles
        torch.cuda.empty_cache()
    return rows


def kernel_short_name(name):
    """A kernel's unqualified name without template arguments ("(anonymous
    namespace)" would otherwise end the name at its parenthesis)."""
    return name.replace("(anonymous namespace)", "~").split("(")[0].split("<")[0].split("::")[-1].split()[-1]


def trace_summary(db):
    """Per-kernel and per-dispatch-shape duration table of a rocprofv3
    --kernel-trace database (the rocpd ``kernels`` view)."""
    import collections
    import sqlite3
    rows = sqlite3.connect(db).execute(
        "select name, duration, grid_x, grid_y, workgroup_x, stream from kernels order by start").fetchall()
    by_name, by_shape = collections.defaultdict(list), collections.defaultdict(list)
    by_stream = collections.defaultdict(list)
    for name, dur, gx, gy, wx, stream in rows:
        short = kernel_short_name(name)
        by_name[short].append(dur)
        by_shape[(short, gx, gy, wx)].append(dur)
        by_stream[(short, stream)].append(dur)
    print("| kernel | calls | avg us | min us | max us | total ms |\n|---|---:|---:|---:|---:|---:|")
    for k, d in sorted(by_name.items(), key=lambda kv: -sum(kv[1])):
        print(f"| {k} | {len(d)} | {sum(d) / len(d) / 1e3:.3f} | {min(d) / 1e3:.3f} | {max(d) / 1e3:.3f} | "
              f"{sum(d) / 1e6:.3f} |")
    print("\nPer stream (the per-shape timings run on a stream of their own, each decode shape "
          "the same number of times):\n\n| kernel | stream | calls | avg us |\n|---|---|---:|---:|")
    for (k, st), d in sorted(by_stream.items()):
        if k.startswith(("gemm_", "linear_", "quant_", "wide_")):
            print(f"| {k} | {st} | {len(d)} | {sum(d) / len(d) / 1e3:.3f} |")
    # One decode GEMM call = one gemm_decode_kernel or gemm_wide_kernel
    # dispatch, or one gemm_prefill_cols_kernel dispatch split along K (grid
    # y > 1: the 64-row tile down_proj runs at 33-64 rows), plus the
    # wide_reduce_kernel that follows a call splitting K over workgroups (as
    # pmc_summary counts them).
    calls, total = collections.Counter(), collections.Counter()
    for name, dur, gx, gy, wx, stream in rows:
        k = kernel_short_name(name)
        is_call = k in ("gemm_decode_kernel", "gemm_wide_kernel") or (k == "gemm_prefill_cols_kernel" and gy > 1)
        if is_call:
            calls[stream] += 1
        if is_call or k == "wide_reduce_kernel":
            total[stream] += dur
    for st in sorted(calls):
        print(f"| decode GEMM per call (gemm_decode_kernel / gemm_wide_kernel / split gemm_prefill_cols_kernel + "
              f"wide_reduce_kernel) | {st} | {calls[st]} | {total[st] / calls[st] / 1e3:.3f} |")
    print("\n| kernel | grid x (threads) | grid y | workgroup | calls | avg us |\n|---|---:|---:|---:|---:|---:|")
    for (k, gx, gy, wx), d in sorted(by_shape.items()):
        if k.startswith(("gemm_", "linear_", "quant_", "wide_", "compat_", "repack_")):
            print(f"| {k} | {gx} | {gy} | {wx} | {len(d)} | {sum(d) / len(d) / 1e3:.3f} |")


def pmc_summary(fetch_db, write_db, out_json=None):
    """HBM bytes per decode GEMM launch from a --pmc-probe run's FETCH_SIZE and
    WRITE_SIZE counters (KiB per dispatch), each scaled by what it reads for the
    probe's closing 256 MiB device copy."""
    import sqlite3

    def load(db, counter):
        return sqlite3.connect(db).execute(
            "select name, counter_value from pmc_events where counter_name=? order by dispatch_id",
            (counter,)).fetchall()

    fetch, write = load(fetch_db, "FETCH_SIZE"), load(write_db, "WRITE_SIZE")
    is_copy = lambda n: "copy" in n.lower()
    cal_kib = 256 * 1024
    ff = cal_kib / [v for n, v in fetch if is_copy(n)][-1]
    fw = cal_kib / [v for n, v in write if is_copy(n)][-1]
    def per_call(events):
        # a call = its gemm_decode_kernel / gemm_wide_kernel dispatch (the probe's
        # only prefill-kernel dispatches are down_proj's split 64-row tiles) plus the
        # wide_reduce_kernel that follows it when K is split over workgroups
        out = []
        for n, v in events:
            if "gemm_decode_kernel" in n or "gemm_wide_kernel" in n or "gemm_prefill_cols_kernel" in n:
                out.append(v)
            elif "wide_reduce_kernel" in n and out:
                out[-1] += v
        return out[-16:]

    gf, gw = per_call(fetch), per_call(write)
    shapes = [(M, p) for M in DECODE_MS for p in PROJS]
    import __graft_entry__ as ge
    synth = ge.package().synth
    print(f"Calibration: the probe's 256 MiB copy reads FETCH_SIZE {cal_kib / ff:.0f} KiB (factor {ff:.4f}) and "
          f"WRITE_SIZE {cal_kib / fw:.0f} KiB (factor {fw:.4f}).\n")
    print("| M | proj | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM MB | algorithmic MB | ratio |\n"
          "|---:|---|---:|---:|---:|---:|---:|")
    out, tot_alg, tot_tr = [], 0.0, 0.0
    for (M, p), f, w in zip(shapes, gf, gw):
        K, N = synth.QWQ_SHAPES[p]
        alg = gemm_bytes(M, N, K)
        tr = f * 1024 * ff + w * 1024 * fw
        tot_alg += alg
        tot_tr += tr
        out.append(dict(M=M, proj=p, fetch_kib=f, write_kib=w, hbm_bytes=round(tr), alg_bytes=alg,
                        ratio=round(tr / alg, 4)))
        print(f"| {M} | {p} | {f:.1f} | {w:.1f} | {tr / 1e6:.3f} | {alg / 1e6:.3f} | {tr / alg:.3f} |")
    n = len(out)
    print(f"\nAverage per launch: {tot_tr / n / 1e6:.3f} MB HBM vs {tot_alg / n / 1e6:.3f} MB algorithmic "
          f"({tot_tr / tot_alg:.3f}x).")
    if out_json:
        with open(out_json, "w") as fh:
            json.dump(dict(factor_fetch=ff, factor_write=fw, per_shape=out, avg_traffic_bytes=tot_tr / n,
                           avg_alg_bytes=tot_alg / n), fh, indent=1)


def int8_library_ref(dev, synth, M, time_graph, prefill):
    """hipBLASLt's int8 x int8 -> int32 GEMM (torch._int_mm) at the four projections' shapes and
    M rows, two weight copies alternating, back-to-back graph replays; beside this build's W4A8
    GEMM at the same M."""
    import torch
    out = {"kernel": "torch._int_mm (hipBLASLt): int8 A [M, K] x int8 W [K, N] -> int32, no group scales",
           "M": M, "shapes": {}}
    ours = {r["proj"]: r for r in prefill if r["M"] == M}
    for p in PROJS:
        K, N = synth.QWQ_SHAPES[p]
        try:
            gen = torch.Generator(device=dev)
            gen.manual_seed(11)
            a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=gen)
            ws = [torch.randint(-8, 8, (N, K), dtype=torch.int8, device=dev, generator=gen).t() for _ in range(2)]

            def mms(a=a, ws=ws, T=6):
                for i in range(T):
                    torch._int_mm(a, ws[i % 2])

            us = time_graph(mms) / 6
            tops = 2 * M * N * K / us / 1e6
            row = {"us": round(us, 2), "TOPS": round(tops, 1), "mfma_frac": round(tops / INT8_PEAK_TOPS, 4)}
            if p in ours:
                row["w4a8_gemm_us"] = ours[p]["gemm_us"]
                row["w4a8_speed_vs_int8"] = round(us / ours[p]["gemm_us"], 3)
            out["shapes"][p] = row
            log(f"  int8 library GEMM {p:13s} M={M:5d}: {us:9.1f} us {tops:7.1f} TOPS ({tops / INT8_PEAK_TOPS:.1%} of "
                f"int8 peak); W4A8 GEMM at {row.get('w4a8_speed_vs_int8', float('nan')):.2f}x its speed")
            del a, ws
        except (RuntimeError, AttributeError) as ex:
            out["shapes"][p] = {"error": f"{type(ex).__name__}: {str(ex)[:160]}"}
    return out


def decode_pmc_summary(dbs):
    """Counter table of the 16 configs[1] decode GEMM calls of a --pmc-probe run: counter
    databases (one pass each), then a --kernel-trace database of the same probe for the
    durations.  A call's counters are those of its GEMM dispatch (gemm_decode_kernel,
    gemm_wide_kernel or the split gemm_prefill_cols_kernel); the wide_reduce_kernel of the
    K-split calls is left out."""
    import collections
    import sqlite3
    *pmc_dbs, trace_db = dbs
    import __graft_entry__ as ge
    synth = ge.package().synth
    is_gemm = lambda n: any(k in n for k in ("gemm_decode_kernel", "gemm_wide_kernel",  # noqa: E731
                                             "gemm_prefill_cols_kernel"))
    short = lambda n: n.split("<")[0].split("::")[-1].replace("void ", "")  # noqa: E731
    shapes = [(M, p) for M in DECODE_MS for p in PROJS]
    calls = [(n, d) for n, d in sqlite3.connect(trace_db).execute(
        "select name, duration from kernels order by start").fetchall() if is_gemm(n)][-len(shapes):]
    ctr = [collections.defaultdict(list) for _ in shapes]
    for db in pmc_dbs:
        ev = sqlite3.connect(db).execute("select dispatch_id, name, counter_name, counter_value from pmc_events "
                                         "order by dispatch_id").fetchall()
        ids = sorted({did for did, name, _, _ in ev if is_gemm(name)})[-len(shapes):]
        pos = {did: i for i, did in enumerate(ids)}
        for did, _, cname, val in ev:
            if did in pos:
                ctr[pos[did]][cname].append(val)
    avg = lambda v: sum(v) / len(v) if v else float("nan")  # noqa: E731
    print("Commands (run from /tmp with TMPDIR=/tmp; REPO is the repository root; one database per run):\n")
    for i, db in enumerate(pmc_dbs):
        names_db = [r[0] for r in sqlite3.connect(db).execute(
            "select distinct counter_name from pmc_events order by counter_name")]
        print(f"    rocprofv3 --pmc {' '.join(names_db)} -d /tmp/dp -o p{i + 1} -- python3 REPO/bench.py --pmc-probe")
    print("    rocprofv3 --kernel-trace -d /tmp/dp -o kt -- python3 REPO/bench.py --pmc-probe")
    print("    python3 REPO/bench.py --decode-pmc-summary " +
          " ".join(f"p{i + 1}_results.db" for i in range(len(pmc_dbs))) + " kt_results.db\n")
    names = sorted({c for d in ctr for c in d})
    print("Per-dispatch values as rocprofv3 reports them (SQ_* per shader engine, 32 on MI355X; "
          "GRBM_GUI_ACTIVE in GPU cycles).\n")
    print("| M | proj | kernel | us | " + " | ".join(names) + " |")
    print("|---:|---|---|---:|" + "---:|" * len(names))
    for (M, p), (n, d), cd in zip(shapes, calls, ctr):
        print(f"| {M} | {p} | {short(n)} | {d / 1e3:.2f} | " + " | ".join(f"{avg(cd[c]):.4g}" for c in names) + " |")

    def frac(cd, a, b):
        try:
            return f"{100 * avg(cd[a]) / avg(cd[b]):.0f}%"
        except ZeroDivisionError:
            return "n/a"
    print("\nDerived: issue and wait shares of the waves' resident cycles (SQ_ACTIVE_INST_ANY, SQ_WAIT_INST_ANY "
          "over SQ_WAVE_CYCLES), VALU instructions per MFMA ((SQ_INSTS_VALU - SQ_INSTS_MFMA) / SQ_INSTS_MFMA), "
          "MFMA busy (SQ_VALU_MFMA_BUSY_CYCLES over 32 SIMDs per shader engine x SQ_BUSY_CYCLES), "
          "SQ_BUSY_CYCLES / duration (the clock while waves are resident; GRBM_GUI_ACTIVE's window is "
          "longer than these few-microsecond dispatches) and the weight stream (algorithmic bytes / duration, "
          "eager calls under the profiler).\n")
    print("| M | proj | issue | wait | VALU / MFMA | MFMA busy | SQ busy GHz | GB/s |\n|---:|---|---:|---:|---:|---:|---:|---:|")
    for (M, p), (n, d), cd in zip(shapes, calls, ctr):
        K, N = synth.QWQ_SHAPES[p]
        g = lambda c: avg(cd[c])  # noqa: E731
        vpm = (g("SQ_INSTS_VALU") - g("SQ_INSTS_MFMA")) / g("SQ_INSTS_MFMA") if g("SQ_INSTS_MFMA") else float("nan")
        busy = 100 * g("SQ_VALU_MFMA_BUSY_CYCLES") / (32 * g("SQ_BUSY_CYCLES"))
        print(f"| {M} | {p} | {frac(cd, 'SQ_ACTIVE_INST_ANY', 'SQ_WAVE_CYCLES')} | "
              f"{frac(cd, 'SQ_WAIT_INST_ANY', 'SQ_WAVE_CYCLES')} | {vpm:.1f} | {busy:.1f}% | "
              f"{g('SQ_BUSY_CYCLES') / d:.2f} | {gemm_bytes(M, N, K) / d:.0f} |")


def prefill_probe(pkg, dev, M, calls=3):
    """Each projection's prefill GEMM at M rows, `calls` times on distinct weight copies
    (eager, group 128, activations drawn on the device), then a 256 MiB copy.  Before every
    call a 512 MiB device copy evicts the caches (the 256 MB Infinity Cache included), so
    the GEMM reads its weights from HBM, as the bench's cold rotation does."""
    import torch
    synth = pkg.synth
    gen = torch.Generator(device=dev)
    fsrc = torch.empty(512 * 2 ** 20, dtype=torch.uint8, device=dev)
    fdst = torch.empty_like(fsrc)
    for pi, p in enumerate(PROJS):
        K, N = synth.QWQ_SHAPES[p]
        x = synth.activations_device(M, K, seed=M + pi, device=dev)
        a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x, GROUP)
        for c in range(calls):
            gen.manual_seed(77 + 10 * pi + c)
            codes = torch.randint(-8, 8, (N, K), dtype=torch.int8, device=dev, generator=gen)
            ws = (torch.rand((K // GROUP, N), device=dev, generator=gen) * 0.018 + 0.002).to(torch.float16)
            wt, st = torch.ops.npu.w4a8_repack(pkg.packing.pack_int4(codes), ws, K, GROUP)
            del codes
            fdst.copy_(fsrc)
            torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP)
            torch.cuda.synchronize()
            del wt, st
        del x, a_q, a_s
    src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"bench: prefill probe done ({len(PROJS)} projections x {calls} calls at M={M}, then a 268435456-byte copy)")


def prefill_pmc_summary(dbs, json_out=None):
    """Counter table of the prefill GEMM (gemm_prefill_kernel or gemm_prefill_cols_kernel) from
    --prefill-probe runs: counter databases
    (one pass each) and a --kernel-trace database (the last argument) for durations."""
    import collections
    import sqlite3
    *pmc_dbs, trace_db = dbs
    import __graft_entry__ as ge
    synth = ge.package().synth
    rows = sqlite3.connect(trace_db).execute(
        "select name, duration, grid_x from kernels order by start").fetchall()
    is_gemm = lambda n: "gemm_prefill_kernel" in n or "gemm_prefill_cols_kernel" in n  # noqa: E731
    gemms = [(d, gx) for n, d, gx in rows if is_gemm(n)]
    kname = sorted({n.split("<")[0].split("::")[-1] for n, _, _ in rows if is_gemm(n)})
    per = max(1, len(gemms) // len(PROJS))
    # the probe's order: each projection's calls in turn (PROJS order); M from
    # the first projection's grid (128 x 128 tiles of 256 threads)
    K0, N0 = synth.QWQ_SHAPES[PROJS[0]]
    M = gemms[0][1] // 256 // -(-N0 // 128) * 128 if gemms else 0
    dur = collections.defaultdict(list)
    for i, (d, gx) in enumerate(gemms):
        dur[PROJS[min(i // per, len(PROJS) - 1)]].append(d)
    ctr = collections.defaultdict(lambda: collections.defaultdict(list))
    cal = {}
    for db in pmc_dbs:
        con = sqlite3.connect(db)
        ev = con.execute("select dispatch_id, name, counter_name, counter_value from pmc_events "
                         "order by dispatch_id").fetchall()
        # the probe's dispatch order: each projection's GEMM calls in turn (PROJS order)
        gemm_ids = sorted({did for did, name, _, _ in ev if is_gemm(name)})
        per = max(1, len(gemm_ids) // len(PROJS))
        which = {did: PROJS[min(i // per, len(PROJS) - 1)] for i, did in enumerate(gemm_ids)}
        for did, name, cname, val in ev:
            if "copy" in name.lower():
                cal[cname] = val
            elif did in which:
                ctr[which[did]][cname].append(val)
    avg = lambda v: sum(v) / len(v) if v else float("nan")  # noqa: E731
    print(f"{' / '.join(kname)} at M={M}, group 128: per-dispatch counter averages (each counter from its own "
          f"pass; the duration from the kernel-trace run).\n")
    print("Commands (run from /tmp with TMPDIR=/tmp; REPO is the repository root; one database per run):\n")
    for i, db in enumerate(pmc_dbs):
        names_db = [r[0] for r in sqlite3.connect(db).execute(
            "select distinct counter_name from pmc_events order by counter_name")]
        print(f"    rocprofv3 --pmc {' '.join(names_db)} -d /tmp/pf -o p{i + 1} -- "
              f"python3 REPO/bench.py --prefill-probe {M}")
    print(f"    rocprofv3 --kernel-trace -d /tmp/pf -o kt -- python3 REPO/bench.py --prefill-probe {M}")
    print("    python3 REPO/bench.py --prefill-pmc-summary " +
          " ".join(f"p{i + 1}_results.db" for i in range(len(pmc_dbs))) + " kt_results.db" +
          (" --pmc-json REPO/profiles/gemm_prefill_cols_kernel_traffic.json" if json_out else "") + "\n")
    names = sorted({c for p in ctr for c in ctr[p]})
    print("| counter | " + " | ".join(PROJS) + " |\n|---|" + "---:|" * len(PROJS))
    print("| duration us | " + " | ".join(f"{avg(dur[p]) / 1e3:.1f}" for p in PROJS) + " |")
    for c in names:
        print(f"| {c} | " + " | ".join(f"{avg(ctr[p][c]):.4g}" for p in PROJS) + " |")
    print("\nDerived (per dispatch):\n\n| metric | " + " | ".join(PROJS) + " |\n|---|" + "---:|" * len(PROJS))
    def row(label, f):
        vals = []
        for p in PROJS:
            try:
                vals.append(f(p))
            except (KeyError, ZeroDivisionError, TypeError):
                vals.append("n/a")
        print(f"| {label} | " + " | ".join(v if isinstance(v, str) else f"{v:.4g}" for v in vals) + " |")
    c = lambda p, n: avg(ctr[p][n])  # noqa: E731
    us = lambda p: avg(dur[p]) / 1e3  # noqa: E731
    row("TOPS (2MNK / duration)", lambda p: 2 * M * synth.QWQ_SHAPES[p][1] * synth.QWQ_SHAPES[p][0] / us(p) / 1e6)
    row("TOPS from 32 x SQ_INSTS_VALU_MFMA_MOPS_I8 x 512", lambda p: 32 * c(p, "SQ_INSTS_VALU_MFMA_MOPS_I8") * 512 / us(p) / 1e6)
    row("VALU instructions per MFMA (SQ_INSTS_VALU - SQ_INSTS_MFMA) / SQ_INSTS_MFMA",
        lambda p: (c(p, "SQ_INSTS_VALU") - c(p, "SQ_INSTS_MFMA")) / c(p, "SQ_INSTS_MFMA"))
    row("LDS instructions per MFMA", lambda p: c(p, "SQ_INSTS_LDS") / c(p, "SQ_INSTS_MFMA"))
    # the counter table holds per-dispatch values as rocprofv3 reduces them:
    # SQ_* counters per shader engine (32 on MI355X: the instruction totals
    # are these times 32, checked against 2*M*N*K below), GRBM_GUI_ACTIVE in
    # GPU cycles
    row("clock GHz (GRBM_GUI_ACTIVE / duration)", lambda p: c(p, "GRBM_GUI_ACTIVE") / us(p) / 1e3)
    row("MFMA busy % (32 x SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x 1024 SIMDs))",
        lambda p: 100 * 32 * c(p, "SQ_VALU_MFMA_BUSY_CYCLES") / (c(p, "GRBM_GUI_ACTIVE") * 1024))
    row("VALU-MFMA co-execution % of MFMA busy", lambda p: 100 * c(p, "SQ_VALU_MFMA_COEXEC_CYCLES") /
        c(p, "SQ_VALU_MFMA_BUSY_CYCLES"))
    if "FETCH_SIZE" in cal and "WRITE_SIZE" in cal:
        ff, fw = 256 * 1024 / cal["FETCH_SIZE"], 256 * 1024 / cal["WRITE_SIZE"]
        row("HBM MB (FETCH_SIZE + WRITE_SIZE, scaled by the 256 MiB copy)",
            lambda p: (c(p, "FETCH_SIZE") * ff + c(p, "WRITE_SIZE") * fw) * 1024 / 1e6)
        row("algorithmic MB", lambda p: gemm_bytes(M, synth.QWQ_SHAPES[p][1], synth.QWQ_SHAPES[p][0]) / 1e6)
        print(f"\nCalibration: the 256 MiB copy reads FETCH_SIZE {cal['FETCH_SIZE']:.0f} KiB (factor {ff:.4f}) and "
              f"WRITE_SIZE {cal['WRITE_SIZE']:.0f} KiB (factor {fw:.4f}).")
        if json_out:
            per = {p: {"traffic_bytes": (c(p, "FETCH_SIZE") * ff + c(p, "WRITE_SIZE") * fw) * 1024,
                       "alg_bytes": gemm_bytes(M, synth.QWQ_SHAPES[p][1], synth.QWQ_SHAPES[p][0]),
                       "duration_us": us(p)} for p in PROJS}
            Path(json_out).write_text(json.dumps(dict(
                kernel=" / ".join(kname), M=M, group=128, factor_fetch=ff, factor_write=fw, per_shape=per,
                avg_traffic_bytes=sum(v["traffic_bytes"] for v in per.values()) / len(per),
                avg_alg_bytes=sum(v["alg_bytes"] for v in per.values()) / len(per)), indent=1) + "\n")


def cpu_baseline(pkg, dev, seconds):
    """The reference's CPU path on configs[0] (o_proj, M=16, K=N=5120, G=128), timed on
    this host, and checked against the GPU output on the same inputs.

    Protocol: the process is pinned to a fixed set of cores (at most 16, the
    host share of one GPU on the box) and the reference's OpenMP team is set to
    that many threads; five timed batches of about seconds/5 each follow one
    untimed run, and the median batch gives the time per linear."""
    import numpy as np
    import torch

    from oracle import ref as oref
    from oracle import w4a8 as ow

    synth = pkg.synth
    M, K, N = 16, 5120, 5120
    xb = synth.activations(M, K, seed=0)
    w = synth.weight_codes_uniform(N, K, 1)
    sb = synth.group_scales(N, K // GROUP, 2, "f16")
    ws32 = synth.scale_bits_to_f32(sb, "f16")

    # GPU on the same inputs
    w_q = torch.from_numpy(ow.pack_grouped(w, GROUP)).to(dev)
    w_scale = torch.from_numpy(np.ascontiguousarray(sb.T).view(np.int16)).view(torch.float16).to(dev)
    wt, st = torch.ops.npu.w4a8_repack(w_q, w_scale, K, GROUP)
    a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev))
    y_gpu = torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP).view(torch.int16).cpu().numpy().view(np.uint16)

    q_ref, s_ref = ow.quant_act_per_token(xb)
    y32 = ow.gemm_fp32(q_ref, s_ref, w, ws32, GROUP)
    fail, n_fb = ow.output_bar(y_gpu, y32, lambda r, c: ow.gemm_f64(q_ref[r], s_ref[r], w[c], ws32[c], GROUP))
    yg = ow.bf16_bits_to_f32(y_gpu).astype(np.float64)
    rb = ow.round_bf16(y32).astype(np.float64)
    parity = {"within_bar": bool(not fail.any()), "float64_fallbacks": n_fb,
              "rel_l2_vs_bf16_oracle": float(np.linalg.norm(yg - rb) / np.linalg.norm(rb)),
              "equal_frac": float(np.mean(yg == rb)),
              "quant_codes_equal": bool(np.array_equal(a_q.cpu().numpy(), q_ref))}

    # pin: the first `cores` CPUs this process may run on
    allowed = sorted(os.sched_getaffinity(0))
    cores = max(1, min(16, len(allowed)))
    pinned = set(allowed[:cores])
    os.sched_setaffinity(0, pinned)
    nbytes = gemm_bytes(M, N, K)
    if oref.available():
        kind = "reference"
        threads = oref.set_threads(cores)
        G = K // GROUP
        wsb = ow.f32_to_bf16_bits(ws32).T.copy()     # the reference C++ takes bf16 group scales

        def run():
            # activation quant (oracle port; the reference's C++ quantiser needs ACL) + reference GEMM
            q, s = ow.quant_act_per_token(xb)
            oref.midgroup_gemm(q, np.repeat(s[None, :], G, axis=0), w, wsb, GROUP)
        what = ("reference C++ ReferenceMidGroupGemm (int4_cube_lab/host/gemm_ref.cpp, OpenMP, built by "
                "oracle/Makefile) + per-token quant (numpy port: the reference's C++ quantiser needs ACL), "
                "configs[0]: o_proj M=16 K=N=5120 G=128")
    else:
        kind = "port"
        threads = torch.get_num_threads()

        def run():
            q, s = ow.quant_act_per_token(xb)
            ow.gemm_fp32(q, s, w, ws32, GROUP)
        what = "numpy restatement (oracle/w4a8.py) of the reference torch CPU path, configs[0]"

    def timed(fn, budget, batches=5):
        """Median seconds per call over `batches` batches of about budget/batches each."""
        fn()
        t0 = time.perf_counter()
        fn()
        one = max(time.perf_counter() - t0, 1e-6)
        per = max(1, int(budget / batches / one))
        times = []
        for _ in range(batches):
            t0 = time.perf_counter()
            for _ in range(per):
                fn()
            times.append((time.perf_counter() - t0) / per)
        return float(np.median(times)), per * batches, times

    try:
        sec, reps, times = timed(run, seconds)
        out = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
               "sample": (f"{what}; pinned to CPUs {min(pinned)}-{max(pinned)} with {threads} threads, median of 5 "
                          f"batches ({reps} runs), {sec * 1e3:.2f} ms per linear"),
               "us_per_linear": round(sec * 1e6, 1),
               "batch_ms": [round(t * 1e3, 2) for t in times], "parity_vs_gpu": parity}
        if kind == "reference":
            # the numpy restatement of the same path, for comparison (numpy's own threading)
            def port():
                q, s = ow.quant_act_per_token(xb)
                ow.gemm_fp32(q, s, w, ws32, GROUP)
            psec, preps, _ = timed(port, max(1.0, seconds / 4))
            out["port"] = {"us_per_linear": round(psec * 1e6, 1), "GBs": round(nbytes / psec / 1e9, 3),
                           "sample": f"oracle/w4a8.py numpy restatement, median of 5 batches ({preps} runs)"}
    finally:
        os.sched_setaffinity(0, set(allowed))
    return out


def gpu_clocks():
    """The GPU's current clock readings from rocm-smi (run as a child process), or None."""
    import subprocess
    try:
        r = subprocess.run(["rocm-smi", "--showclocks", "--json"], capture_output=True, text=True, timeout=30)
        card = next(iter(json.loads(r.stdout).values()))
        return {k.rstrip(":"): v for k, v in card.items() if "clk" in k.lower() and "speed" in k.lower()}
    except Exception:   # tool missing or output not JSON: the clocks are informational only
        return None


if __name__ == "__main__":
    main()
