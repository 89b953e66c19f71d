#!/usr/bin/env python3
"""W4A8 per-group linear throughput at QwQ-32B shapes on one MI355X.

Metric: "W4A8 GEMM TOPS + weight GB/s (% roofline), QwQ-32B
shapes, M=1..4096".

One step = the decode configuration: dynamic per-token int8
quant + W4A8 GEMM for each QwQ-32B projection (qkv 5120->7168, o 5120->5120,
gate_up 5120->55296, down 27648->5120) at M in {1, 4, 16, 64}, group 128 --
16 linears.  Weights are rotated over distinct copies totalling >= 1 GiB so
that every step streams them from HBM, not from the 256 MB Infinity Cache
(the reference's cold protocol, int4_cube_lab/host/mg_harness.h:42, :215-219).
Each step is replayed as a HIP graph (one per weight copy).

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
    ap.add_argument("--prefill-m", default="1024,4096")
    ap.add_argument("--no-detail", action="store_true", help="only the timed steps (for profiling)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: each decode linear once (eager) on cold weights, then a "
                         "256 MiB device copy of known size for calibrating the byte counters")
    args = ap.parse_args()
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

    # ---------------------------------------------------------------- data
    per_set = sum(synth.QWQ_SHAPES[p][0] * synth.QWQ_SHAPES[p][1] // 2 for p in PROJS)
    copies = max(2, math.ceil(args.cold_bytes * 2 ** 30 / per_set))
    log(f"bench: {props.name}, {copies} weight copies x {per_set / 1e6:.0f} MB")
    gen = torch.Generator(device=dev)
    weights = {}
    for pi, p in enumerate(PROJS):
        K, N = synth.QWQ_SHAPES[p]
        weights[p] = []
        for r in range(copies):
            gen.manual_seed(1000 * pi + r)
            codes = torch.randint(-8, 8, (N, K), dtype=torch.int8, device=dev, generator=gen)
            w_q = pkg.packing.pack_int4(codes)
            del codes
            ws = (torch.rand((K // GROUP, N), device=dev, generator=gen) * 0.018 + 0.002).to(torch.float16)
            weights[p].append(torch.ops.npu.w4a8_repack(w_q, ws, K, GROUP))
            del w_q, ws
    xs = {}
    for M in DECODE_MS:
        for p in PROJS:
            K, _ = synth.QWQ_SHAPES[p]
            xb = synth.activations(M, K, seed=10 * M + PROJS.index(p))
            xs[(M, p)] = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)
    torch.cuda.synchronize()

    def step(r):
        outs = []
        for M in DECODE_MS:
            for p in PROJS:
                K, N = synth.QWQ_SHAPES[p]
                wt, st = weights[p][r]
                a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(xs[(M, p)])
                outs.append(torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP))
        return outs

    if args.pmc_probe:
        for i, M in enumerate(DECODE_MS):
            for j, p in enumerate(PROJS):
                K, N = synth.QWQ_SHAPES[p]
                wt, st = weights[p][(i * len(PROJS) + j) % copies]
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
        for r in range(copies):      # warm the capture stream (workspace is allocated here, not in capture)
            step(r)
    torch.cuda.current_stream(dev).wait_stream(cap)
    torch.cuda.synchronize()
    graphs = []
    for r in range(copies):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            step(r)
        graphs.append(g)
    torch.cuda.synchronize()

    bytes_per_step = sum(gemm_bytes(M, synth.QWQ_SHAPES[p][1], synth.QWQ_SHAPES[p][0]) +
                         quant_bytes(M, synth.QWQ_SHAPES[p][0]) for M in DECODE_MS for p in PROJS)

    # ---------------------------------------------------------------- timed region
    for i in range(args.warmup):
        graphs[i % copies].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        graphs[(args.warmup + i) % copies].replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
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
                               "M in {1,4,16,64}, group 128, cold (weights rotated over "
                               f"{copies} copies = {copies * per_set / 2 ** 30:.2f} GiB)",
                   "group": GROUP, "linears_per_step": len(DECODE_MS) * len(PROJS),
                   "bytes_per_step": bytes_per_step},
    }
    if args.no_detail:
        print(json.dumps(result), flush=True)
        return

    # ---------------------------------------------------------------- per-shape kernel times
    T = args.detail_launches
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

    def time_graph(fn, reps=3):
        with torch.cuda.stream(cap):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            fn()
        g.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            e0, e1 = ev(), ev()
            e0.record()
            g.replay()
            e1.record()
            e1.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3)   # us
        del g
        return sorted(times)[len(times) // 2]

    shapes = []
    tot_bytes = tot_us = 0.0
    for M in DECODE_MS:
        for p in PROJS:
            K, N = synth.QWQ_SHAPES[p]
            a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(xs[(M, p)])

            def gemms(a_q=a_q, a_s=a_s, p=p, K=K, N=N):
                for i in range(T):
                    wt, st = weights[p][i % copies]
                    torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP)

            def quants(M=M, p=p):
                for _ in range(T):
                    torch.ops.npu.w4a8_quant_pertoken(xs[(M, p)])

            us = time_graph(gemms) / T
            qus = time_graph(quants) / T
            b = gemm_bytes(M, N, K)
            tot_bytes += b
            tot_us += us
            shapes.append({"proj": p, "M": M, "N": N, "K": K, "gemm_us": round(us, 3),
                           "gemm_GBs": round(b / us / 1e3, 1), "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                           "TOPS": round(2 * M * N * K / us / 1e6, 2), "quant_us": round(qus, 3)})
            log(f"  {p:13s} M={M:3d}: gemm {us:8.2f} us {b / us / 1e3:7.1f} GB/s ({b / us / 1e3 / HBM_PEAK_GBS:.1%})"
                f"  quant {qus:6.2f} us")
    achieved = tot_bytes / tot_us / 1e3
    # HBM bytes per launch from the two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) recorded in
    # profiles/ (the command is in the summary), each scaled by a 256 MiB copy's reading.
    traffic, traffic_src = None, ROOT / "profiles" / "gemm_decode_kernel_traffic.json"
    if traffic_src.exists():
        traffic = round(json.loads(traffic_src.read_text())["avg_traffic_bytes"])
    result["roofline"] = {
        "kernel": "gemm_decode_kernel (decode W4A8 GEMM, all 16 configs[1] shapes, cold)",
        "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
        "per_launch_bytes_avg": round(tot_bytes / len(shapes)), "launch_us_avg": round(tot_us / len(shapes), 3),
        "timing": "HIP events around graph replays of back-to-back launches on the launch stream",
        "traffic_source": str(traffic_src.relative_to(ROOT)) if traffic is not None else None,
    }
    result["decode_shapes"] = shapes

    # ---------------------------------------------------------------- prefill
    prefill = []
    for M in [int(m) for m in args.prefill_m.split(",") if m]:
        for p in PROJS:
            K, N = synth.QWQ_SHAPES[p]
            x = torch.from_numpy(synth.activations(M, K, seed=M).view(np.int16)).view(torch.bfloat16).to(dev)
            a_q, a_s = torch.ops.npu.w4a8_quant_pertoken(x)
            Tp = max(2, min(10, int(2e4 // max(1, M))))

            def gemms(a_q=a_q, a_s=a_s, p=p, K=K, N=N, Tp=Tp):
                for i in range(Tp):
                    wt, st = weights[p][i % copies]
                    torch.ops.npu.w4a8_gemm(a_q, a_s, wt, st, N, K, GROUP)

            us = time_graph(gemms) / Tp
            tops = 2 * M * N * K / us / 1e6
            prefill.append({"proj": p, "M": M, "gemm_us": round(us, 2), "TOPS": round(tops, 1),
                            "mfma_frac": round(tops / INT8_PEAK_TOPS, 4)})
            log(f"  prefill {p:13s} M={M:5d}: {us:9.1f} us {tops:7.1f} TOPS ({tops / INT8_PEAK_TOPS:.1%} of int8 peak)")
            del x, a_q, a_s
    result["prefill_shapes"] = prefill

    # ---------------------------------------------------------------- CPU baseline
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(pkg, dev, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def cpu_baseline(pkg, dev, seconds):
    """The reference's CPU path on configs[0] (o_proj, M=16, K=N=5120, G=128), timed on
    this host, and checked against the GPU output on the same inputs."""
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
    y32, mag = ow.gemm_fp32(q_ref, s_ref, w, ws32, GROUP, return_abs=True)
    yg = ow.bf16_bits_to_f32(y_gpu).astype(np.float64)
    tol = ow.bf16_ulp(y32) + 2 * ow.fp32_sum_error_bound(mag, K // GROUP)
    rb = ow.round_bf16(y32).astype(np.float64)
    parity = {"within_bound": bool(np.all(np.abs(yg - y32) <= tol)),
              "rel_l2_vs_bf16_oracle": float(np.linalg.norm(yg - rb) / np.linalg.norm(rb)),
              "equal_frac": float(np.mean(yg == rb)),
              "quant_codes_equal": bool(np.array_equal(a_q.cpu().numpy(), q_ref))}

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    nbytes = gemm_bytes(M, N, K)
    if oref.available():
        kind = "reference"
        G = K // GROUP
        asg = np.repeat(s_ref[None, :], G, axis=0)
        wsb = ow.f32_to_bf16_bits(ws32).T.copy()     # the reference C++ takes bf16 group scales

        def run():
            # activation quant (oracle port; the reference's C++ quantiser needs ACL) + reference GEMM
            q, s = ow.quant_act_per_token(xb)
            oref.midgroup_gemm(q, np.repeat(s[None, :], G, axis=0), w, wsb, GROUP)
        what = ("reference C++ ReferenceMidGroupGemm (int4_cube_lab/host/gemm_ref.cpp, OpenMP, built by "
                "oracle/Makefile) + per-token quant, configs[0]: o_proj M=16 K=N=5120 G=128")
        del asg
    else:
        kind = "port"

        def run():
            q, s = ow.quant_act_per_token(xb)
            ow.gemm_fp32(q, s, w, ws32, GROUP)
        what = "numpy restatement (oracle/w4a8.py) of the reference torch CPU path, configs[0]"
    run()
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 10000:
            break
    sec = el / reps
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"{what}; {reps} runs in {el:.1f} s, {sec * 1e3:.2f} ms per linear",
            "us_per_linear": round(sec * 1e6, 1), "parity_vs_gpu": parity}


if __name__ == "__main__":
    main()
