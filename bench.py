#!/usr/bin/env python3
"""Decode hot-path benchmark on one MI355X.

Headline (one JSON line on stdout): Q4_0 mat-vec GB/s over one Llama-3-8B-shaped layer's seven GGML_OP_MUL_MAT
ops at ne11 = 1 (Wq 4096x4096, Wk/Wv 1024x4096, Wo 4096x4096, gate/up 14336x4096, down 4096x14336), each a full
op (Q8_1 quantization of src1 + integer mat-vec) as ggml runs it. A step is one layer; steps rotate over 8
distinct layers of weights (982 MB > the 256 MB Infinity Cache) and run as a replayed HIP graph, so host launch
cost is outside the timed GPU work. Bytes per op follow the reference's mm-gbps formula
(bin/mm-gbps.py:51-57): M*K/32*18 + n*K*4 + M*n*4.

Also reported: the dominant kernel's roofline (the Q4_0 4096x14336 mat-vec, its duration from HIP events around
single launches), FA decode at ctx 8192 (32/8 heads, d 128, fp16 K/V) in microseconds with its roofline, the
Q4_0/Q8_0 sweep at ne11 in {1,2,4,8}, a kernel-sum estimate of 8B-shape decode tokens/s, and the CPU oracle
timed on this host as the baseline.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

PEAK_GBS = 8000.0  # MI355X HBM3E
LAYER = [("wq", 4096, 4096), ("wk", 1024, 4096), ("wv", 1024, 4096), ("wo", 4096, 4096),
         ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
METRIC = "Q4_0 matvec GB/s (% HBM peak); FA-decode µs @ctx 8K; 8B-shape decode tok/s"


def matvec_bytes(wtype, M, K, n):
    blk, nbytes = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}[wtype]
    return M * K // blk * nbytes + n * K * 4 + M * n * 4


def fa_bytes(hq, hkv, ctx, d):
    return 2 * hkv * ctx * d * 2 + 2 * hq * d * 4


class Timer:
    """Per-launch HIP event pairs on torch's current stream, each behind a GPU spacer so that the measured
    interval is the kernel itself rather than host launch latency."""

    def __init__(self, torch):
        self.torch = torch
        self.spacer = torch.empty(64 << 20, dtype=torch.float32, device="cuda")  # 256 MB memset, ~40 us

    def per_launch_us(self, fn, reps):
        torch = self.torch
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for i, (a, b) in enumerate(pairs):
            self.spacer.zero_()
            a.record()
            fn(i)
            b.record()
        torch.cuda.synchronize()
        times = sorted(a.elapsed_time(b) * 1000.0 for a, b in pairs)
        return sum(times) / len(times), times[len(times) // 2]


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8, help="distinct weight sets rotated over steps")
    ap.add_argument("--kernel-reps", type=int, default=100)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bounded CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline and roofline only")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a HIP graph")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path runs on a single "
              "MI355X, see DESIGN.md for how it would shard)", file=sys.stderr)
        sys.exit(2)

    import torch

    import p100_amd as P
    from p100_amd import synth

    lib = P.load()
    torch.manual_seed(0)
    dev = torch.device("cuda")
    stream = torch.cuda.current_stream()
    sp = C.c_void_p(stream.cuda_stream)
    log = lambda *a: print(*a, file=sys.stderr, flush=True)
    log(f"[bench] {torch.cuda.get_device_name(0)}; building {args.layers} Q4_0 layers")

    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    layers = [{name: synth.random_weights(P.Q4_0, M, K, generator=gen) for name, M, K in LAYER}
              for _ in range(args.layers)]
    xs = {4096: torch.randn(4096, device=dev, generator=gen), 14336: torch.randn(14336, device=dev, generator=gen)}
    ys = {name: torch.empty(M, device=dev) for name, M, K in LAYER}
    ws_bytes = lib.p1x_mul_mat_vec_workspace(P.Q4_0, 14336, 14336, 8, 0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()

    def run_layer(layer):
        sp = C.c_void_p(torch.cuda.current_stream().cuda_stream)  # the capture stream while capturing
        for name, M, K in LAYER:
            rc = lib.p1x_mul_mat_vec(P.Q4_0, C.c_void_p(layer[name].data_ptr()), K // 32 * 18, M, K, 0,
                                     C.c_void_p(xs[K].data_ptr()), 1, C.c_void_p(ys[name].data_ptr()), None,
                                     C.c_void_p(ws.data_ptr()), ws_bytes, sp)
            if rc:
                raise RuntimeError(lib.p1x_last_error().decode())

    step_bytes = sum(matvec_bytes(P.Q4_0, M, K, 1) for _, M, K in LAYER)
    # Eager reference outputs for the graph check.
    run_layer(layers[0])
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in ys.items()}

    launch = "eager"
    graphs = None
    if not args.eager:
        try:
            graphs = []
            for li in range(args.layers):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    run_layer(layers[li])
                graphs.append(g)
            # Every replay must reproduce the eager result (no memset nodes; checked, not assumed).
            for _ in range(3):
                for y in ys.values():
                    y.fill_(float("nan"))
                graphs[0].replay()
                torch.cuda.synchronize()
                for k, v in ys.items():
                    if not torch.equal(v, eager[k]):
                        raise RuntimeError(f"graph replay differs from eager for {k}")
            launch = "hip-graph"
        except Exception as e:  # fall back to eager launches, and say so in the JSON
            log(f"[bench] graph capture unavailable ({e}); timing eager launches")
            graphs = None
    stream = torch.cuda.current_stream()
    sp = C.c_void_p(stream.cuda_stream)

    def step(i):
        if graphs is not None:
            graphs[i % args.layers].replay()
        else:
            run_layer(layers[i % args.layers])

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(args.steps):
        step(i)
    t1.record()
    torch.cuda.synchronize()
    ms_total = t0.elapsed_time(t1)
    ms_per_step = ms_total / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"[bench] layer step {ms_per_step * 1e3:.2f} us, {value:.1f} GB/s ({launch})")

    # Dominant kernel: Q4_0 4096x14336 mat-vec on a prepared Q8_1 activation, single launches.
    timer = Timer(torch)
    q81 = P.quantize_q8_1(xs[14336])
    ydown = torch.empty(4096, device=dev)

    def down(i):
        w = layers[i % args.layers]["down"]
        lib.p1x_mul_mat_vec_q8_1(P.Q4_0, C.c_void_p(w.data_ptr()), 14336 // 32 * 18, 4096, 14336,
                                 C.c_void_p(q81.qs.data_ptr()), C.c_void_p(q81.ds.data_ptr()), 1,
                                 C.c_void_p(ydown.data_ptr()), None, sp)

    k_avg, k_med = timer.per_launch_us(down, args.kernel_reps)
    k_bytes = matvec_bytes(P.Q4_0, 4096, 14336, 1)
    achieved = k_bytes / (k_avg * 1e-6) / 1e9
    log(f"[bench] Q4_0 4096x14336 mat-vec kernel avg {k_avg:.2f} us (median {k_med:.2f}) -> {achieved:.0f} GB/s")

    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 (q4_0 x q8_1 dot4, int32 sums, fp32 scales)", "data": "synthetic",
        "config": {"workload": "Llama-3-8B layer mat-vec sweep, Q4_0, ne11=1: Wq 4096x4096, Wk/Wv 1024x4096, "
                               "Wo 4096x4096, gate/up 14336x4096, down 4096x14336; weights N(0,0.02) quantized "
                               "with ggml's q4_0 reference rule, x N(0,1); 8 weight sets rotated (982 MB)",
                   "op": "quantize_q8_1 + mul_mat_vec per matrix", "launch": launch,
                   "bytes_per_step": step_bytes, "pct_hbm_peak": round(100 * value / PEAK_GBS, 2)},
        "roofline": {"kernel": "k_mmvq<q4_0,1> 4096x14336", "bound": "hbm", "achieved": round(achieved, 1),
                     "peak": PEAK_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": k_bytes, "avg_us": round(k_avg, 3), "median_us": round(k_med, 3)},
    }

    if not args.no_extra:
        result["extra"] = extra_measurements(torch, P, lib, synth, timer, sp, gen, log, args)

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, P, layers[0]["down"], xs[14336], args.cpu_seconds, log)
    print(json.dumps(result), flush=True)


def extra_measurements(torch, P, lib, synth, timer, sp, gen, log, args):
    dev = torch.device("cuda")
    out = {}
    # FA decode: 32/8 heads, d 128, 1 query row; 16 KV caches rotated (537 MB at ctx 8192).
    fa = {}
    for ctx in (512, 2048, 8192, 32768):
        p = P.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=ctx, d_qk=128, d_v=128, causal=True)
        nsets = max(1, min(16, (600 << 20) // (2 * 8 * ctx * 128 * 2)))
        caches = [(torch.randn(8 * ctx * 128, device=dev, generator=gen).half(),
                   torch.randn(8 * ctx * 128, device=dev, generator=gen).half()) for _ in range(nsets)]
        q = torch.randn(32 * 128, device=dev, generator=gen)
        o = torch.empty(32 * 128, device=dev)
        lse = torch.empty(32, device=dev)
        need = P.flash_attn_decode_workspace(p)
        ws = torch.empty(need // 4 + 4, dtype=torch.float32, device=dev)

        def call(i, p=p, caches=caches, q=q, o=o, lse=lse, ws=ws, need=need):
            k, v = caches[i % len(caches)]
            lib.p1x_flash_attn_decode(C.byref(p), C.c_void_p(q.data_ptr()), C.c_void_p(k.data_ptr()),
                                      C.c_void_p(v.data_ptr()), None, None, C.c_void_p(o.data_ptr()),
                                      C.c_void_p(lse.data_ptr()), C.c_void_p(ws.data_ptr()), ws.numel() * 4, sp)

        call(0)
        torch.cuda.synchronize()
        avg, med = timer.per_launch_us(call, max(20, args.kernel_reps // 2))
        b = fa_bytes(32, 8, ctx, 128)
        fa[str(ctx)] = {"us": round(avg, 3), "median_us": round(med, 3), "bytes": b,
                        "gbs": round(b / (avg * 1e-6) / 1e9, 1), "frac": round(b / (avg * 1e-6) / 1e9 / PEAK_GBS, 4)}
        log(f"[bench] FA decode ctx {ctx}: {avg:.2f} us ({fa[str(ctx)]['gbs']} GB/s)")
        del caches
    out["fa_decode"] = {"config": "32 q heads / 8 kv heads, d 128, 1 query row, causal, fp16 K/V, fp32 out+lse; "
                                  "split-K + LSE combine (2 kernels, timed together)", "by_ctx": fa}

    # Per-op sweep (quantize + mat-vec), Q4_0 and Q8_0, ne11 in {1,2,4,8}, 4 rotated weight sets each.
    sweep = {}
    for wtype, tname in ((P.Q4_0, "q4_0"), (P.Q8_0, "q8_0")):
        for name, M, K in (("wq", 4096, 4096), ("wk", 1024, 4096), ("gate", 14336, 4096), ("down", 4096, 14336)):
            nsets = max(2, min(8, (600 << 20) // (M * K)))
            ws_ = [synth.random_weights(wtype, M, K, generator=gen) for _ in range(nsets)]
            for n in (1, 2, 4, 8):
                x = torch.randn((n, K), device=dev, generator=gen)
                y = torch.empty((n, M), device=dev)
                wsz = lib.p1x_mul_mat_vec_workspace(wtype, M, K, n, 0)
                wsb = torch.empty(wsz, dtype=torch.uint8, device=dev)
                rb = P.row_bytes(wtype, K)

                def call(i, ws_=ws_, x=x, y=y, wsb=wsb, wsz=wsz, M=M, K=K, n=n, wtype=wtype, rb=rb):
                    lib.p1x_mul_mat_vec(wtype, C.c_void_p(ws_[i % len(ws_)].data_ptr()), rb, M, K, 0,
                                        C.c_void_p(x.data_ptr()), n, C.c_void_p(y.data_ptr()), None,
                                        C.c_void_p(wsb.data_ptr()), wsz, sp)

                avg, med = timer.per_launch_us(call, 30)
                b = matvec_bytes(wtype, M, K, n)
                sweep[f"{tname} {M}x{K} n={n}"] = {"us": round(avg, 3), "gbs": round(b / (avg * 1e-6) / 1e9, 1)}
            del ws_
    out["matvec_sweep_op_us"] = sweep
    log("[bench] sweep: " + ", ".join(f"{k}: {v['gbs']}" for k, v in sweep.items() if k.endswith("n=1")))

    # 8B-shape decode tokens/s, summed from measured op times: 32 x (7 Q4_0 ops + FA @ ctx 640) + Q4_0 output
    # projection 128256x4096. No norm/RoPE/SwiGLU/KV-append glue; an estimate, not an end-to-end run.
    wout = [synth.random_weights(P.Q4_0, 128256, 4096, generator=gen) for _ in range(2)]
    x = torch.randn(4096, device=dev, generator=gen)
    y = torch.empty(128256, device=dev)
    wsz = lib.p1x_mul_mat_vec_workspace(P.Q4_0, 128256, 4096, 1, 0)
    wsb = torch.empty(wsz, dtype=torch.uint8, device=dev)

    def outproj(i):
        lib.p1x_mul_mat_vec(P.Q4_0, C.c_void_p(wout[i % 2].data_ptr()), 4096 // 32 * 18, 128256, 4096, 0,
                            C.c_void_p(x.data_ptr()), 1, C.c_void_p(y.data_ptr()), None, C.c_void_p(wsb.data_ptr()),
                            wsz, sp)

    out_us, _ = timer.per_launch_us(outproj, 20)
    layer_ops = {}
    for name, M, K in LAYER:
        key = f"q4_0 {M}x{K} n=1"
        layer_ops[name] = sweep[key]["us"] if key in sweep else None
    layer_ops["wv"] = layer_ops["wk"]
    layer_ops["wo"] = layer_ops["wq"]
    layer_ops["up"] = layer_ops["gate"]
    p = P.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=640, d_qk=128, d_v=128, causal=True)
    k = torch.randn(8 * 640 * 128, device=dev, generator=gen).half()
    v = torch.randn(8 * 640 * 128, device=dev, generator=gen).half()
    q = torch.randn(32 * 128, device=dev, generator=gen)
    o = torch.empty(32 * 128, device=dev)
    ws = torch.empty(P.flash_attn_decode_workspace(p) // 4 + 4, device=dev)

    def fa640(i):
        lib.p1x_flash_attn_decode(C.byref(p), C.c_void_p(q.data_ptr()), C.c_void_p(k.data_ptr()),
                                  C.c_void_p(v.data_ptr()), None, None, C.c_void_p(o.data_ptr()), None,
                                  C.c_void_p(ws.data_ptr()), ws.numel() * 4, sp)

    fa_us, _ = timer.per_launch_us(fa640, 20)
    token_us = 32 * (sum(layer_ops.values()) + fa_us) + out_us
    token_bytes = 32 * sum(matvec_bytes(P.Q4_0, M, K, 1) for _, M, K in LAYER) + fa_bytes(32, 8, 640, 128) * 32 \
        + matvec_bytes(P.Q4_0, 128256, 4096, 1)
    out["decode_8b_kernel_sum"] = {
        "tok_s": round(1e6 / token_us, 1), "us_per_token": round(token_us, 1),
        "roofline_tok_s": round(PEAK_GBS * 1e9 / token_bytes, 1), "output_proj_us": round(out_us, 2),
        "note": "sum of measured single-op times: 32 x (7 Q4_0 mat-vec ops + FA decode @ctx 640) + Q4_0 "
                "128256x4096 output projection; excludes norm/RoPE/SwiGLU/KV-append glue and launch gaps"}
    log(f"[bench] 8B decode kernel-sum estimate {1e6 / token_us:.1f} tok/s")
    return out


def cpu_baseline(torch, P, w_dev, x_dev, seconds, log):
    """The CPU oracle's Q8_1 integer mat-vec (OpenMP over rows) on the same 4096x14336 Q4_0 matrix and input,
    repeated for about `seconds` seconds on this host; reported in GB/s with the same byte count."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import numpy as np

    import oracle

    w = w_dev.cpu().numpy()
    x = x_dev.cpu().numpy().reshape(1, -1)
    M, K = 4096, 14336
    oracle.mul_mat_vec(P.Q4_0, w, M, K, x)  # warm-up
    n, t0 = 0, time.perf_counter()
    times = []
    while time.perf_counter() - t0 < seconds or n < 3:
        a = time.perf_counter()
        oracle.mul_mat_vec(P.Q4_0, w, M, K, x)
        times.append(time.perf_counter() - a)
        n += 1
    times.sort()
    med = times[len(times) // 2]
    b = matvec_bytes(P.Q4_0, M, K, 1)
    threads = oracle.max_threads()
    cpu = "unknown"
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                cpu = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    log(f"[bench] CPU oracle q4_0 4096x14336: {med * 1e3:.2f} ms median over {n} runs, {threads} threads")
    return {"value": round(b / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"Q4_0 4096x14336 ne11=1 op (Q8_1 quantize + integer dot), {n} runs in {sum(times):.1f} s, "
                      f"median {med * 1e3:.2f} ms; scalar C++ restatement, OpenMP over rows; {cpu}"}


if __name__ == "__main__":
    main()
