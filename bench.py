#!/usr/bin/env python3
"""Decode hot-path benchmark on one MI355X.

Headline (one JSON line on stdout): Q4_0 mat-vec GB/s over one Llama-3-8B-shaped layer's seven GGML_OP_MUL_MAT
ops at ne11 = 1 (Wq 4096x4096, Wk/Wv 1024x4096, Wo 4096x4096, gate/up 14336x4096, down 4096x14336), each a full
op (Q8_1 quantization of src1 + integer mat-vec) as ggml runs it. A step is one layer; steps rotate over 8
distinct layers of weights (982 MB > the 256 MB Infinity Cache) and run as a replayed HIP graph, so host launch
cost is outside the timed GPU work. Bytes per op follow the reference's mm-gbps formula
(bin/mm-gbps.py:51-57): M*K/32*18 + n*K*4 + M*n*4.

Kernel figures (the roofline of the dominant kernel, FA decode, the sweep) are per-launch periods of graphs of
back-to-back launches over rotated buffers, timed with HIP events on the launching stream: with the queue full
the launch gap is small, so the period tracks the kernel's own duration (compare profiles/).

Also reported: FA decode at ctx 512..32768 (32/8 heads, d 128, fp16 K/V), the Q4_0/Q8_0 sweep at ne11 in
{1,2,4,8}, the layer step with one shared Q8_1 preparation per input (q/k/v and gate/up share theirs), a
kernel-sum estimate of 8B-shape decode tokens/s, and the CPU oracle timed on this host as the baseline.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import pathlib
import sys
import time

PEAK_GBS = 8000.0  # MI355X HBM3E
LAYER = [("wq", 4096, 4096), ("wk", 1024, 4096), ("wv", 1024, 4096), ("wo", 4096, 4096),
         ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
ROWS = {name: M for name, M, _ in LAYER}
METRIC = "Q4_0 matvec GB/s (% HBM peak); FA-decode µs @ctx 8K; 8B-shape decode tok/s"


def matvec_bytes(wtype, M, K, n):
    blk, nbytes = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}[wtype]
    return M * K // blk * nbytes + n * K * 4 + M * n * 4


def fa_bytes(hq, hkv, ctx, d):
    return 2 * hkv * ctx * d * 2 + 2 * hq * d * 4


def rotation(set_bytes, total=544 << 20, cap=256):
    """Distinct buffer sets to rotate over so that the sets one timed graph touches span > 512 MB (twice the
    256 MB Infinity Cache): each launch then reads bytes the previous ~512 MB of traffic has evicted. The graph
    holds max(32, sets) launches so that every set is read."""
    return max(2, min(cap, -(-total // set_bytes)))


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def ok(lib, rc, what):
    """Every timed C-ABI call is checked: a rejected call enqueues nothing, and an empty replay must not be timed."""
    if rc:
        raise RuntimeError(f"{what}: p1x error {rc}: {lib.p1x_last_error().decode()}")


class GraphTimer:
    """Per-launch period of `n` back-to-back launches captured in one HIP graph (launch i gets index i, so the
    callee can rotate buffers), timed with HIP events around replays on the current stream."""

    def __init__(self, torch):
        self.torch = torch

    def stream(self):
        return C.c_void_p(self.torch.cuda.current_stream().cuda_stream)

    def period_us(self, fn, n=64, replays=5):
        torch = self.torch
        fn(0, self.stream())  # eager warm-up (and first-use initialisation) outside the capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            s = self.stream()
            for i in range(n):
                fn(i, s)
        g.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(replays):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) * 1000.0 / n)
        times.sort()
        return times[len(times) // 2], times[0], times[-1]


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--layers", type=int, default=8, help="distinct weight sets rotated over steps")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bounded CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline and roofline only")
    ap.add_argument("--only", choices=("roofline", "fa", "decode", "cols", "kquant", "read", "mmvh"), default=None,
                    help="run one measurement alone (for profiler runs whose per-kernel averages must not mix "
                         "shapes): 'roofline' = the Q4_0 4096x14336 mat-vec, 'fa' = FA decode at --fa-ctx, "
                         "'decode' = the end-to-end 8B greedy decode, 'cols' = the Q4_0 4096x14336 mat-vec on a "
                         "prepared Q8_1 activation of --cols columns, 'kquant' = the K-quant kernels (--kquant "
                         "picks one shape), 'read' = the read-ceiling probe, 'mmvh' = the h16 kernels")
    ap.add_argument("--kquant", default=None, help="with --only kquant: one of q4_K:14336x4096, q4_K:4096x14336, "
                                                     "q6_K:128256x4096")
    ap.add_argument("--mmvh", default=None, help="with --only mmvh: one TYPE:MxK of the h16 comparison (e.g. "
                                                   "q4_K:4096x14336)")
    ap.add_argument("--cols", type=int, nargs="+", default=[4, 16])
    ap.add_argument("--fa-ctx", type=int, nargs="+", default=[512, 640, 2048, 8192, 32768])
    ap.add_argument("--tbo-sql", default=None, metavar="PATH",
                    help="also write the mat-vec sweep and the FA legs as test-backend-ops perf rows (the SQL that "
                         "the reference's bin/mm-gbps.py and bench/analyze.py read)")
    ap.add_argument("--fa-kernel", choices=("auto", "split", "mc"), default="auto",
                    help="first-pass attention kernel (p1x_fa_select_kernel): the automatic choice, the vector "
                         "pass, or the matrix-core alternative")
    ap.add_argument("--fa-fp16-only", action="store_true",
                    help="with --only fa: the fp16 cache at --fa-ctx alone (no device-length or quantized-cache "
                         "runs), so a profile of the run holds one configuration")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: this decode path runs on a "
              "single MI355X (tensor-parallel sharding of the weight rows is not built)", file=sys.stderr)
        sys.exit(2)

    import torch

    import p100_amd as P
    from p100_amd import synth

    lib = P.load()
    P.fa_select_kernel(args.fa_kernel)
    dev = torch.device("cuda")
    if args.only == "decode":
        print(json.dumps({"only": "decode", "decode_8b": measure_decode(torch)}))
        return
    if args.only == "cols":
        gen = torch.Generator(device="cuda")
        gen.manual_seed(77)
        M, K = 4096, 14336
        wsets = [synth.random_weights(P.Q4_0, M, K, generator=gen) for _ in range(8)]
        timer = GraphTimer(torch)
        rec = {}
        for n in args.cols:
            q = P.quantize_q8_1(torch.randn((n, K), device=dev, generator=gen))
            y = torch.empty((n, M), device=dev)

            def call(i, s, q=q, y=y, n=n):
                rc = lib.p1x_mul_mat_vec_q8_1(P.Q4_0, C.c_void_p(wsets[i % 8].data_ptr()), K // 32 * 18, M, K,
                                              C.c_void_p(q.qs.data_ptr()), C.c_void_p(q.ds.data_ptr()), n,
                                              C.c_void_p(y.data_ptr()), None, s)
                if rc:
                    raise RuntimeError(lib.p1x_last_error().decode())

            med, mn, _ = timer.period_us(call, n=32)
            b = matvec_bytes(P.Q4_0, M, K, n)
            rec[str(n)] = {"us": round(med, 3), "min_us": round(mn, 3), "gbs": round(b / (med * 1e-6) / 1e9, 1)}
            log(f"[bench] Q4_0 {M}x{K} at {n} columns (prepared Q8_1): {med:.2f} us")
        print(json.dumps({"only": "cols", "q4_0_4096x14336_prepared": rec}))
        return
    if args.only in ("kquant", "read", "mmvh"):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(99)
        timer = GraphTimer(torch)
        if args.only == "read":
            print(json.dumps({"only": "read", "read_ceiling": measure_read_ceiling(torch, lib, timer)}))
        elif args.only == "kquant":
            print(json.dumps({"only": "kquant", "kquant": measure_kquant(torch, P, lib, synth, timer, gen,
                                                                         args.kquant)}))
        else:
            print(json.dumps({"only": "mmvh", "mmvh": measure_mmvh(torch, P, lib, synth, timer, gen, args.mmvh)}))
        return
    log(f"[bench] {torch.cuda.get_device_name(0)}; building {args.layers} Q4_0 layers")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    layers = [{name: synth.random_weights(P.Q4_0, M, K, generator=gen) for name, M, K in LAYER}
              for _ in range(args.layers)]
    xs = {4096: torch.randn(4096, device=dev, generator=gen), 14336: torch.randn(14336, device=dev, generator=gen)}
    ys = {name: torch.empty(M, device=dev) for name, M, K in LAYER}
    ws_bytes = lib.p1x_mul_mat_vec_workspace(P.Q4_0, 14336, 14336, 8, 0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    timer = GraphTimer(torch)
    torch.cuda.synchronize()
    if args.only == "roofline":
        roof = measure_roofline(torch, P, lib, timer, gen, xs[14336])
        # Calibration for hardware byte counters: a plain 32 MiB device copy (reads and writes 33,554,432 B).
        src = torch.empty(32 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"only": "roofline", "roofline": roof, "calibration_copy_bytes": 32 << 20}))
        return
    if args.only == "fa":
        rec = {"only": "fa", "fa_decode": measure_fa(torch, P, lib, timer, gen, args.fa_ctx,
                                                     kvlen_runs=not args.fa_fp16_only)}
        for kv_type in () if args.fa_fp16_only else ("q8_0", "q4_0"):
            rec[f"fa_decode_{kv_type}_kv"] = measure_fa_quant(torch, P, lib, synth, timer, gen, args.fa_ctx, kv_type)
        if args.tbo_sql:
            write_tbo_sql(args.tbo_sql, rec, torch.cuda.get_device_name(0))
        print(json.dumps(rec))
        return

    def op(wt, M, K, x, y, s):
        rc = lib.p1x_mul_mat_vec(P.Q4_0, C.c_void_p(wt.data_ptr()), K // 32 * 18, M, K, 0, C.c_void_p(x.data_ptr()),
                                 1, C.c_void_p(y.data_ptr()), None, C.c_void_p(ws.data_ptr()), ws_bytes, s)
        if rc:
            raise RuntimeError(lib.p1x_last_error().decode())

    def layer_step(i, s):
        layer = layers[i % args.layers]
        for name, M, K in LAYER:
            op(layer[name], M, K, xs[K], ys[name], s)

    # A captured layer must reproduce the eager result bit for bit on every replay (no memset nodes).
    layer_step(0, timer.stream())
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in ys.items()}
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        layer_step(0, timer.stream())
    for _ in range(3):
        for y in ys.values():
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        g1.replay()
        torch.cuda.synchronize()
        for k, v in ys.items():
            if not torch.equal(v, eager[k]):
                raise RuntimeError(f"graph replay differs from eager for {k}")

    # Timed: graphs of n_graph consecutive layer steps over the rotated weight sets.
    step_bytes = sum(matvec_bytes(P.Q4_0, M, K, 1) for _, M, K in LAYER)
    n_graph = max(d for d in range(1, min(args.steps, 64) + 1) if args.steps % d == 0)  # exactly K steps timed
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = timer.stream()
        for i in range(n_graph):
            layer_step(i, s)
    for _ in range(max(1, -(-args.warmup // n_graph))):
        g.replay()
    torch.cuda.synchronize()
    replays = args.steps // n_graph
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(replays):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    steps_done = replays * n_graph
    ms_per_step = t0.elapsed_time(t1) / steps_done
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"[bench] layer step {ms_per_step * 1e3:.2f} us, {value:.1f} GB/s ({steps_done} steps in graphs of {n_graph})")

    roof = measure_roofline(torch, P, lib, timer, gen, xs[14336])

    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps_done,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 (q4_0 x q8_1 dot4, int32 sums, fp32 scales)", "data": "synthetic",
        "config": {"workload": "Llama-3-8B layer mat-vec sweep, Q4_0, ne11=1: Wq 4096x4096, Wk/Wv 1024x4096, "
                               "Wo 4096x4096, gate/up 14336x4096, down 4096x14336; weights N(0,0.02) quantized "
                               "with ggml's q4_0 reference rule, x N(0,1); 8 weight sets rotated (982 MB)",
                   "op": "p1x_mul_mat_vec per matrix: one launch with in-kernel Q8_1 for Wq/Wk/Wv/Wo, Q8_1 "
                         "quantize + mat-vec for gate/up/down (10 launches per step)", "launch": "hip-graph",
                   "bytes_per_step": step_bytes, "pct_hbm_peak": round(100 * value / PEAK_GBS, 2)},
        "roofline": roof,
    }
    if not args.no_extra:
        result["extra"] = extra_measurements(torch, P, lib, synth, timer, gen, layers, xs, args.fa_ctx)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(P, layers[0]["down"], xs[14336], args.cpu_seconds)
    if args.tbo_sql:
        write_tbo_sql(args.tbo_sql, result.get("extra", {}), torch.cuda.get_device_name(0))
    print(json.dumps(result), flush=True)


# test-backend-ops perf rows (the schema of the reference's tests/fixtures/tbo-perf-cpu.sql:1-18), so that the
# reference's own analysis scripts read this bench: MUL_MAT cases keyed by type_a, m, n, k with an unbatched,
# contiguous f32 right-hand side (bin/mm-gbps.py:24-31), FLASH_ATTN_EXT cases in test-backend-ops' parameter
# spelling. time_us is the measured graph period of the op; memory_kb the algorithmic bytes.
TBO_COLUMNS = ("test_time", "build_commit", "backend_name", "op_name", "op_params", "test_mode", "supported",
               "passed", "error_message", "time_us", "flops", "bandwidth_gb_s", "memory_kb", "n_runs",
               "device_description", "backend_reg_name")


def tbo_rows(extra):
    """(op_name, op_params, time_us, bytes, flops) for each mat-vec sweep point and FA context in `extra`."""
    rows = []
    ops = dict(extra.get("matvec_sweep_op_us", {}))  # "q4_0 4096x14336 n=1": {"us", ...}
    # The K-quant legs' whole op (Q8_1 pass + kernel), the quantity test-backend-ops times; kernel-only entries
    # (prepared activation) are not test-backend-ops rows.
    ops.update({k: v["op"] for k, v in extra.get("kquant", {}).items() if "op" in v})
    for key, rec in ops.items():
        tname, shape, ncols = key.split()
        m, k = (int(v) for v in shape.split("x"))
        n = int(ncols.split("=")[1])
        blk, per = {"q4_0": (18, 32), "q8_0": (34, 32), "q4_K": (144, 256), "q6_K": (210, 256)}[tname]
        nbytes = m * k // per * blk + n * k * 4 + m * n * 4  # bin/mm-gbps.py:51-57
        params = (f"type_a={tname},type_b=f32,m={m},n={n},k={k},bs=[1,1],nr=[1,1],per=[0,1,2,3],k_v=0,o=1,"
                  "src_overlap=0,m_v=0,pad=0")
        rows.append(("MUL_MAT", params, rec["us"], nbytes, 2.0 * m * n * k))
    for name, kv_type in (("fa_decode", "f16"), ("fa_decode_q8_0_kv", "q8_0"), ("fa_decode_q4_0_kv", "q4_0")):
        for ctx, rec in extra.get(name, {}).get("by_ctx", {}).items():
            kv = int(ctx)
            params = (f"hsk=128,hsv=128,nh=8,nr23=[4,1],kv={kv},nb=1,mask=0,sinks=0,max_bias=0.000000,"
                      f"logit_softcap=0.000000,prec=f32,type_K={kv_type},type_V={kv_type},permute=[0,1,2,3],"
                      "kv_view=0,v_is_view_of_k=0,n_kv_max=0")
            rows.append(("FLASH_ATTN_EXT", params, rec["us"], rec.get("bytes", 0), 4.0 * 32 * 128 * kv))
    return rows


def write_tbo_sql(path, extra, device):
    import datetime

    now = datetime.datetime.now(datetime.timezone.utc).strftime("%Y-%m-%dT%H:%M:%SZ")
    kinds = {"supported": "INTEGER", "passed": "INTEGER", "memory_kb": "INTEGER", "n_runs": "INTEGER",
             "time_us": "REAL", "flops": "REAL", "bandwidth_gb_s": "REAL"}
    lines = ["CREATE TABLE IF NOT EXISTS test_backend_ops (",
             ",\n".join(f"  {c} {kinds.get(c, 'TEXT')}" for c in TBO_COLUMNS), ");", ""]
    for op, params, us, nbytes, flops in tbo_rows(extra):
        vals = (now, "p100_amd", "ROCm0", op, params, "perf", "1", "1", "", f"{us:.6f}",
                f"{flops / (us * 1e-6):.6f}", f"{nbytes / (us * 1e-6) / 1e9:.6f}", str(nbytes // 1024), "1",
                device, "ROCm")
        lines.append(f"INSERT INTO test_backend_ops ({', '.join(TBO_COLUMNS)}) VALUES "
                     f"({', '.join(repr(v) for v in vals)});")
    pathlib.Path(path).write_text("\n".join(lines) + "\n")
    log(f"[bench] wrote {len(lines) - 4} test-backend-ops rows to {path}")


def measure_roofline(torch, P, lib, timer, gen, x):
    """Dominant kernel: the Q4_0 4096x14336 mat-vec on a prepared Q8_1 activation, rotated over 16 weight sets
    (530 MB)."""
    from p100_amd import synth

    M, K = 4096, 14336
    b = matvec_bytes(P.Q4_0, M, K, 1)
    nsets = rotation(M * K // 32 * 18)
    wsets = [synth.random_weights(P.Q4_0, M, K, generator=gen) for _ in range(nsets)]
    q81 = P.quantize_q8_1(x)
    y = torch.empty(M, device=x.device)

    def down(i, s):
        w = wsets[i % nsets]
        ok(lib, lib.p1x_mul_mat_vec_q8_1(P.Q4_0, C.c_void_p(w.data_ptr()), K // 32 * 18, M, K,
                                         C.c_void_p(q81.qs.data_ptr()), C.c_void_p(q81.ds.data_ptr()), 1,
                                         C.c_void_p(y.data_ptr()), None, s), "roofline mat-vec")

    med, mn, _ = timer.period_us(down, n=max(64, nsets))
    del wsets
    achieved = b / (med * 1e-6) / 1e9
    log(f"[bench] Q4_0 4096x14336 mat-vec kernel {med:.2f} us (min {mn:.2f}) -> {achieved:.0f} GB/s ({nsets} sets)")
    # HBM bytes per launch of this kernel from the FETCH_SIZE / WRITE_SIZE profiler passes (calibrated against a
    # 32 MiB copy), recorded next to the rocprof summary; null when that record is absent.
    traffic, src = None, None
    rec = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    if os.path.exists(rec):
        with open(rec) as f:
            t = json.load(f).get("k_mmvr q4_0 4096x14336 ne11=1")
        if t:
            traffic, src = t["traffic_bytes"], t["source"]
    return {"kernel": "k_mmvr<q4_0> 4096x14336 (prepared Q8_1 activation held in registers; row-groups of 4 waves "
                      "x 4 rows, 2 units per lane)", "bound": "hbm",
            "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_GBS, 4),
            "traffic": traffic, "traffic_unit": "bytes per launch", "traffic_source": src,
            "algorithmic_bytes": b, "avg_us": round(med, 3), "min_us": round(mn, 3),
            "rotation": f"{nsets} weight sets, {nsets * M * K // 32 * 18 / 1e6:.0f} MB"}


def measure_read_ceiling(torch, lib, timer, nbytes=33103872 // 16 * 16):
    """The single-launch read ceiling: p1x_read_bytes over the roofline kernel's byte count, rotated over > 512 MB,
    for several grid sizes; the fastest is the ceiling any one kernel reading these bytes once can reach."""
    nsets = rotation(nbytes)
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i) for i in range(nsets)]
    digest = torch.empty(65536, dtype=torch.int32, device="cuda")
    by_grid = {}
    for wgs in (1024, 2048, 4096, 8192):
        def call(i, s, wgs=wgs):
            ok(lib, lib.p1x_read_bytes(C.c_void_p(bufs[i % nsets].data_ptr()), nbytes, C.c_void_p(digest.data_ptr()),
                                       wgs, s), "read_bytes")

        med, mn, _ = timer.period_us(call, n=max(64, nsets))
        by_grid[str(wgs)] = {"us": round(med, 3), "gbs": round(nbytes / (med * 1e-6) / 1e9, 1)}
    del bufs
    best = min(by_grid, key=lambda k: by_grid[k]["us"])
    us = by_grid[best]["us"]
    log(f"[bench] read ceiling {nbytes / 1e6:.1f} MB: {us:.2f} us ({nbytes / (us * 1e-6) / 1e9:.0f} GB/s, "
        f"{best} work-groups)")
    return {"bytes": nbytes, "us": us, "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_GBS, 4), "work_groups": int(best), "by_grid": by_grid,
            "kernel": "k_read_bytes: non-temporal 16-byte loads, 4 in flight per thread, grid-stride, one launch",
            "rotation": f"{nsets} buffers, {nsets * nbytes / 1e6:.0f} MB"}


def measure_matvec(torch, P, lib, synth, timer, gen, wtype, M, K, ncols, act="q8_1", prepared=True):
    """Per-launch period of one mat-vec shape over > 512 MB of rotated weights: the prepared-activation kernel
    alone (prepared=True) or the whole op from an f32 activation (quantize / pre-pass + mat-vec)."""
    rb = P.row_bytes(wtype, K)
    nsets = rotation(M * rb)
    wsets = [synth.random_weights(wtype, M, K, generator=gen) for _ in range(nsets)]
    x = torch.randn((ncols, K), device="cuda", generator=gen)
    y = torch.empty((ncols, M), device="cuda")
    if prepared and act == "q8_1":
        a = P.quantize_q8_1(x)

        def call(i, s):
            ok(lib, lib.p1x_mul_mat_vec_q8_1(wtype, C.c_void_p(wsets[i % nsets].data_ptr()), rb, M, K,
                                             C.c_void_p(a.qs.data_ptr()), C.c_void_p(a.ds.data_ptr()), ncols,
                                             C.c_void_p(y.data_ptr()), None, s), "mul_mat_vec_q8_1")
    elif prepared:
        a = P.prepare_h16(x)

        def call(i, s):
            ok(lib, lib.p1x_mul_mat_vec_h16(wtype, C.c_void_p(wsets[i % nsets].data_ptr()), rb, M, K,
                                            C.c_void_p(a.h.data_ptr()), C.c_void_p(a.meta.data_ptr()), ncols,
                                            C.c_void_p(y.data_ptr()), s), "mul_mat_vec_h16")
    else:
        mode = P.ACT[act]
        wsz = lib.p1x_mul_mat_vec_workspace(wtype, M, K, ncols, mode)
        wsb = torch.empty(max(wsz, 256), dtype=torch.uint8, device="cuda")

        def call(i, s):
            ok(lib, lib.p1x_mul_mat_vec(wtype, C.c_void_p(wsets[i % nsets].data_ptr()), rb, M, K, mode,
                                        C.c_void_p(x.data_ptr()), ncols, C.c_void_p(y.data_ptr()), None,
                                        C.c_void_p(wsb.data_ptr()), wsb.numel(), s), "mul_mat_vec")

    med, mn, _ = timer.period_us(call, n=max(32, nsets))
    del wsets
    b = matvec_bytes(wtype, M, K, ncols)
    gbs = b / (med * 1e-6) / 1e9
    return {"us": round(med, 3), "min_us": round(mn, 3), "gbs": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
            "sets": nsets}


def measure_fa(torch, P, lib, timer, gen, ctxs, kvlen_runs=True):
    """FA decode: 32/8 heads, d 128, 1 query row, causal; KV caches rotated beyond the Infinity Cache."""
    dev = torch.device("cuda")
    fa = {}
    for ctx in ctxs:
        p = P.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=ctx, d_qk=128, d_v=128, causal=True)
        nsets = rotation(2 * 8 * ctx * 128 * 2)
        caches = [(torch.randn(8 * ctx * 128, device=dev, generator=gen).half(),
                   torch.randn(8 * ctx * 128, device=dev, generator=gen).half()) for _ in range(nsets)]
        q = torch.randn(32 * 128, device=dev, generator=gen)
        o = torch.empty(32 * 128, device=dev)
        lse = torch.empty(32, device=dev)
        fws = torch.empty(P.flash_attn_decode_workspace(p) // 4 + 4, device=dev)

        def call(i, s, p=p, caches=caches, q=q, o=o, lse=lse, fws=fws):
            k, v = caches[i % len(caches)]
            ok(lib, lib.p1x_flash_attn_decode(C.byref(p), C.c_void_p(q.data_ptr()), C.c_void_p(k.data_ptr()),
                                              C.c_void_p(v.data_ptr()), None, None, C.c_void_p(o.data_ptr()),
                                              C.c_void_p(lse.data_ptr()), C.c_void_p(fws.data_ptr()),
                                              fws.numel() * 4, s), "flash_attn_decode")

        med, mn, _ = timer.period_us(call, n=max(32, nsets))
        b = fa_bytes(32, 8, ctx, 128)
        fa[str(ctx)] = {"us": round(med, 3), "min_us": round(mn, 3), "bytes": b,
                        "gbs": round(b / (med * 1e-6) / 1e9, 1), "frac": round(b / (med * 1e-6) / 1e9 / PEAK_GBS, 4),
                        "sets": nsets}
        log(f"[bench] FA decode ctx {ctx}: {med:.2f} us ({fa[str(ctx)]['gbs']} GB/s)")
        del caches
    # A short visible length in a large cache (device-side length, plan made for the capacity): the kernels spread
    # the visible keys over every planned split, so this should cost what the same length costs on its own.
    cap, kvlen = 8192, {}
    if not kvlen_runs:
        return {"config": "32 q heads / 8 kv heads, d 128, 1 query row, causal, fp16 K/V, fp32 o + lse; split-K "
                          "pass + LSE combine pass (2 launches, timed together)", "by_ctx": fa}
    p = P.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=cap, d_qk=128, d_v=128, causal=True)
    nsets = rotation(2 * 8 * cap * 128 * 2)
    caches = [(torch.randn(8 * cap * 128, device=dev, generator=gen).half(),
               torch.randn(8 * cap * 128, device=dev, generator=gen).half()) for _ in range(nsets)]
    q = torch.randn(32 * 128, device=dev, generator=gen)
    o = torch.empty(32 * 128, device=dev)
    lse = torch.empty(32, device=dev)
    fws = torch.empty(P.flash_attn_decode_workspace(p) // 4 + 4, device=dev)
    n_dev = torch.zeros(1, dtype=torch.int32, device=dev)
    for n in (640, 2048):
        n_dev.fill_(n)

        def call(i, s):
            k, v = caches[i % len(caches)]
            ok(lib, lib.p1x_flash_attn_decode_kvlen(C.byref(p), C.c_void_p(q.data_ptr()), C.c_void_p(k.data_ptr()),
                                                    C.c_void_p(v.data_ptr()), None, None,
                                                    C.c_void_p(n_dev.data_ptr()), C.c_void_p(o.data_ptr()),
                                                    C.c_void_p(lse.data_ptr()), C.c_void_p(fws.data_ptr()),
                                                    fws.numel() * 4, s), "flash_attn_decode_kvlen")

        med, mn, _ = timer.period_us(call, n=max(32, nsets))
        kvlen[str(n)] = {"us": round(med, 3), "min_us": round(mn, 3)}
        log(f"[bench] FA decode, {n} visible keys in a cache of {cap}: {med:.2f} us")
    del caches
    return {"config": "32 q heads / 8 kv heads, d 128, 1 query row, causal, fp16 K/V, fp32 o + lse; split-K pass "
                      "+ LSE combine pass (2 launches, timed together)", "by_ctx": fa,
            "kvlen_cap8192": {"config": "p1x_flash_attn_decode_kvlen over a cache of 8192 rows with the visible "
                                        "length on the device", "by_len": kvlen}}


def measure_fa_quant(torch, P, lib, synth, timer, gen, ctxs, kv_type):
    """FA decode over a q8_0 / q4_0 KV cache (in-kernel dequantization), same shape as measure_fa."""
    dev = torch.device("cuda")
    t = P.TYPES[kv_type]
    row = 128 // 32 * P.BLOCK[t][1]
    fa = {}
    for ctx in ctxs:
        p = P.AttnParams(n_head_q=32, n_head_kv=8, seq_q=1, seq_kv=ctx, d_qk=128, d_v=128, causal=True)
        nsets = rotation(2 * 8 * ctx * row)
        caches = [(synth.random_weights(t, 8 * ctx, 128, std=1.0, generator=gen),
                   synth.random_weights(t, 8 * ctx, 128, std=1.0, generator=gen)) for _ in range(nsets)]
        q = torch.randn(32 * 128, device=dev, generator=gen)
        o = torch.empty(32 * 128, device=dev)
        lse = torch.empty(32, device=dev)
        fws = torch.empty(P.flash_attn_decode_workspace(p) // 4 + 4, device=dev)

        def call(i, s, p=p, caches=caches, q=q, o=o, lse=lse, fws=fws):
            k, v = caches[i % len(caches)]
            ok(lib, lib.p1x_flash_attn_decode_quant(C.byref(p), t, C.c_void_p(q.data_ptr()),
                                                    C.c_void_p(k.data_ptr()), C.c_void_p(v.data_ptr()), None, None,
                                                    None, C.c_void_p(o.data_ptr()), C.c_void_p(lse.data_ptr()),
                                                    C.c_void_p(fws.data_ptr()), fws.numel() * 4, s),
               "flash_attn_decode_quant")

        med, mn, _ = timer.period_us(call, n=max(32, nsets))
        b = 2 * 8 * ctx * row + 32 * 128 * 4 * 2  # quantized K and V once per KV head, q and o in f32
        fa[str(ctx)] = {"us": round(med, 3), "min_us": round(mn, 3), "bytes": b,
                        "gbs": round(b / (med * 1e-6) / 1e9, 1), "frac": round(b / (med * 1e-6) / 1e9 / PEAK_GBS, 4)}
        log(f"[bench] FA decode {kv_type} KV ctx {ctx}: {med:.2f} us ({fa[str(ctx)]['gbs']} GB/s)")
        del caches
    return {"config": f"as fa_decode with a {kv_type} KV cache dequantized in-kernel", "by_ctx": fa}


KQUANT_SHAPES = [("q4_K", 14336, 4096), ("q4_K", 4096, 14336), ("q6_K", 128256, 4096)]


def measure_kquant(torch, P, lib, synth, timer, gen, only=None):
    """The K-quant configuration at ne11 = 1: Q4_K FFN matrices and the Q6_K output projection, as the whole op
    from an f32 activation (Q8_1 quantize + mat-vec) and as the mat-vec kernel on a prepared activation; and the
    kernel at 8 and 16 columns."""
    out = {}
    for tname, M, K in KQUANT_SHAPES:
        key = f"{tname}:{M}x{K}"
        if only and key != only:
            continue
        t = P.TYPES[tname]
        kern = measure_matvec(torch, P, lib, synth, timer, gen, t, M, K, 1, prepared=True)
        op = measure_matvec(torch, P, lib, synth, timer, gen, t, M, K, 1, prepared=False)
        out[f"{tname} {M}x{K} n=1"] = {"kernel": kern, "op": op}
        log(f"[bench] {tname} {M}x{K}: kernel {kern['us']} us ({kern['gbs']} GB/s, frac {kern['frac']}), "
            f"op {op['us']} us")
        # The same matrices at 8 and 16 columns (int8 matrix cores), kernel on a prepared activation.
        for n in (8, 16):
            kn = measure_matvec(torch, P, lib, synth, timer, gen, t, M, K, n, prepared=True)
            out[f"{tname} {M}x{K} n={n}"] = {"kernel": kn}
            log(f"[bench] {tname} {M}x{K} n={n}: kernel {kn['us']} us ({kn['gbs']} GB/s)")
    return out


MMVH_SHAPES = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


def measure_mmvh(torch, P, lib, synth, timer, gen, only=None):
    """The h16 (MMVH) mat-vec kernel against the Q8_1 (MMVQ) kernel on prepared activations, at the Llama-3-8B
    layer shapes, ne11 in {1, 4, 8}: the measurements behind p1x_should_use_mmvh. only = "TYPE:MxK" keeps one."""
    out = {}
    for tname in ("q4_0", "q8_0", "q4_K", "q6_K"):
        t = P.TYPES[tname]
        for M, K in MMVH_SHAPES:
            if only is not None and only != f"{tname}:{M}x{K}":
                continue
            for n in (1, 4, 8):
                h = measure_matvec(torch, P, lib, synth, timer, gen, t, M, K, n, act="h16", prepared=True)
                q = measure_matvec(torch, P, lib, synth, timer, gen, t, M, K, n, act="q8_1", prepared=True)
                out[f"{tname} {M}x{K} n={n}"] = {"h16_us": h["us"], "q8_1_us": q["us"], "h16_gbs": h["gbs"],
                                                  "q8_1_gbs": q["gbs"]}
        if any(k.startswith(tname) for k in out):
            log(f"[bench] mmvh {tname}: " + ", ".join(f"{k.split(' ', 1)[1]} h16 {v['h16_us']} / q8_1 {v['q8_1_us']} us"
                                                    for k, v in out.items() if k.startswith(tname)))
    if only is not None and not out:
        raise SystemExit(f"--mmvh {only}: not one of the measured TYPE:MxK")
    return out


def extra_measurements(torch, P, lib, synth, timer, gen, layers, xs, ctxs):
    dev = torch.device("cuda")
    out = {}
    # Layer step with one Q8_1 preparation per distinct input: x_attn feeds q/k/v, the attention output feeds
    # Wo, x_ffn feeds gate/up, the SwiGLU output feeds down (4 quantizations + 7 mat-vecs = 11 launches).
    acts = {4096: (torch.empty((1, 4096), dtype=torch.int8, device=dev), torch.empty((1, 128, 4), device=dev)),
            14336: (torch.empty((1, 14336), dtype=torch.int8, device=dev), torch.empty((1, 448, 4), device=dev))}
    ys = {name: torch.empty(M, device=dev) for name, M, K in LAYER}

    def quant(K, s):
        qs, ds = acts[K]
        ok(lib, lib.p1x_quantize_q8_1(C.c_void_p(xs[K].data_ptr()), C.c_void_p(qs.data_ptr()),
                                      C.c_void_p(ds.data_ptr()), K, 1, s), "quantize_q8_1")

    def mv(w, M, K, y, s):
        qs, ds = acts[K]
        ok(lib, lib.p1x_mul_mat_vec_q8_1(P.Q4_0, C.c_void_p(w.data_ptr()), K // 32 * 18, M, K,
                                         C.c_void_p(qs.data_ptr()), C.c_void_p(ds.data_ptr()), 1,
                                         C.c_void_p(y.data_ptr()), None, s), "mul_mat_vec_q8_1")

    def shared_step(i, s):
        L = layers[i % len(layers)]
        quant(4096, s)
        for name in ("wq", "wk", "wv"):
            mv(L[name], ROWS[name], 4096, ys[name], s)
        quant(4096, s)
        mv(L["wo"], 4096, 4096, ys["wo"], s)
        quant(4096, s)
        mv(L["gate"], 14336, 4096, ys["gate"], s)
        mv(L["up"], 14336, 4096, ys["up"], s)
        quant(14336, s)
        mv(L["down"], 4096, 14336, ys["down"], s)

    med, mn, mx = timer.period_us(shared_step, n=len(layers) * 4)
    sb = sum(matvec_bytes(P.Q4_0, M, K, 1) for _, M, K in LAYER)
    out["layer_step_shared_q8_1"] = {"us": round(med, 2), "gbs": round(sb / (med * 1e-6) / 1e9, 1), "launches": 11}
    log(f"[bench] layer step, shared Q8_1: {med:.2f} us ({sb / (med * 1e-6) / 1e9:.0f} GB/s)")

    # Per-op sweep (quantize + mat-vec), Q4_0 and Q8_0, ne11 in {1,2,4,8}, rotated weight sets.
    sweep = {}
    for wtype, tname in ((P.Q4_0, "q4_0"), (P.Q8_0, "q8_0")):
        for name, M, K in (("wq", 4096, 4096), ("wk", 1024, 4096), ("gate", 14336, 4096), ("down", 4096, 14336)):
            rb = P.row_bytes(wtype, K)
            nsets = rotation(M * rb)
            wsets = [synth.random_weights(wtype, M, K, generator=gen) for _ in range(nsets)]
            for n in (1, 2, 4, 8, 16):  # 16: the int8 matrix-core form (9..16 columns)
                x = torch.randn((n, K), device=dev, generator=gen)
                y = torch.empty((n, M), device=dev)
                wsz = lib.p1x_mul_mat_vec_workspace(wtype, M, K, n, 0)
                wsb = torch.empty(wsz, dtype=torch.uint8, device=dev)

                def call(i, s, wsets=wsets, x=x, y=y, wsb=wsb, wsz=wsz, M=M, K=K, n=n, wtype=wtype, rb=rb):
                    ok(lib, lib.p1x_mul_mat_vec(wtype, C.c_void_p(wsets[i % len(wsets)].data_ptr()), rb, M, K, 0,
                                                C.c_void_p(x.data_ptr()), n, C.c_void_p(y.data_ptr()), None,
                                                C.c_void_p(wsb.data_ptr()), wsz, s), "mul_mat_vec")

                med, _, _ = timer.period_us(call, n=max(32, nsets))
                b = matvec_bytes(wtype, M, K, n)
                sweep[f"{tname} {M}x{K} n={n}"] = {"us": round(med, 3), "gbs": round(b / (med * 1e-6) / 1e9, 1)}
            del wsets
    out["matvec_sweep_op_us"] = sweep
    log("[bench] sweep n=1: " + ", ".join(f"{k}: {v['us']}us {v['gbs']}" for k, v in sweep.items() if k.endswith("n=1")))

    out["read_ceiling"] = measure_read_ceiling(torch, lib, timer)
    out["kquant"] = measure_kquant(torch, P, lib, synth, timer, gen)
    out["mmvh_vs_mmvq"] = measure_mmvh(torch, P, lib, synth, timer, gen)
    out["fa_decode"] = measure_fa(torch, P, lib, timer, gen, sorted(set(ctxs) | {640}))
    fa = out["fa_decode"]["by_ctx"]
    for kv_type in ("q8_0", "q4_0"):
        out[f"fa_decode_{kv_type}_kv"] = measure_fa_quant(torch, P, lib, synth, timer, gen, (2048, 8192, 32768), kv_type)

    # 8B-shape decode tokens/s from measured periods: 32 x (layer step with shared Q8_1 + FA decode @ctx 640)
    # + Q4_0 output projection 128256x4096. Norm/RoPE/SwiGLU/KV-append glue kernels are not included.
    wout = [synth.random_weights(P.Q4_0, 128256, 4096, generator=gen) for _ in range(2)]
    yo = torch.empty(128256, device=dev)

    def outproj(i, s):
        mv(wout[i % 2], 128256, 4096, yo, s)

    out_us, _, _ = timer.period_us(outproj, n=16)
    token_us = 32 * (out["layer_step_shared_q8_1"]["us"] + fa["640"]["us"]) + out_us
    token_bytes = 32 * (sb + fa_bytes(32, 8, 640, 128)) + matvec_bytes(P.Q4_0, 128256, 4096, 1)
    out["decode_8b_kernel_sum"] = {
        "tok_s": round(1e6 / token_us, 1), "us_per_token": round(token_us, 1),
        "roofline_tok_s": round(PEAK_GBS * 1e9 / token_bytes, 1), "output_proj_us": round(out_us, 2),
        "note": "sum of measured graph periods: 32 x (layer step with shared Q8_1 + FA decode @ctx 640) + Q4_0 "
                "128256x4096 output projection; excludes norm/RoPE/SwiGLU/KV-append glue kernels"}
    log(f"[bench] 8B decode kernel-sum estimate {1e6 / token_us:.1f} tok/s")
    del wout
    out["decode_8b"] = measure_decode(torch)
    return out


def measure_decode(torch, n_prompt=512, n_gen=256, seed=7):
    """End-to-end greedy decode of the random-init Llama-3-8B-shaped Q4_0 model (32 layers, fp16 KV cache):
    the prompt's positions then n_gen decode steps, each step one replay of a captured p1x_llama_decode_step
    graph (a whole token: embedding, 32 layers, output projection, argmax); decode tok/s = n_gen / time."""
    from p100_amd import llama

    hp = llama.hparams(n_prompt + n_gen)
    t_build = time.time()
    model = llama.LlamaModel(hp, device="cuda", seed=seed)
    torch.cuda.synchronize()
    t_build = time.time() - t_build
    dec = llama.Decoder(model, max_prompt=n_prompt)
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, hp.n_vocab, (n_prompt,), generator=g).tolist()
    dec.reset(prompt)
    dec.capture()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    ev[0].record()
    dec.run(n_prompt)
    ev[1].record()
    dec.run(n_gen)
    ev[2].record()
    torch.cuda.synchronize()
    prompt_ms, gen_ms = ev[0].elapsed_time(ev[1]), ev[1].elapsed_time(ev[2])
    state = dec.state.tolist()
    toks = dec.tokens[n_prompt:n_prompt + n_gen + 1].tolist()
    if state[0] != n_prompt + n_gen or not all(0 <= t < hp.n_vocab for t in toks):
        raise RuntimeError(f"decode ended in an unexpected state {state[:3]}")
    kv_read = sum(fa_bytes(hp.n_head, hp.n_head_kv, p + 1, hp.head_dim) for p in range(n_prompt, n_prompt + n_gen))
    token_bytes = model.weight_bytes() + kv_read / n_gen
    us_tok = gen_ms * 1e3 / n_gen
    out = {
        "tok_s": round(n_gen / (gen_ms * 1e-3), 1), "us_per_token": round(us_tok, 1),
        "gbs": round(token_bytes / (us_tok * 1e-6) / 1e9, 1),
        "roofline_tok_s": round(PEAK_GBS * 1e9 / token_bytes, 1), "bytes_per_token": int(token_bytes),
        "prompt_positions_tok_s": round(n_prompt / (prompt_ms * 1e-3), 1),
        "config": f"Llama-3-8B shape (32 layers, 4096, FFN 14336, 32/8 heads x 128, vocab 128256), Q4_0 weights "
                  f"N(0,0.02) random-init, fp16 KV cache; prompt {n_prompt} random ids fed through the decode step, "
                  f"then {n_gen} greedy decode steps timed; one HIP graph per token replayed",
        "launches_per_token": 1 + hp.n_layer * 8 + 4,  # embed; per layer q/k/v (norm inside), FA x2, o, norm,
        # gate/up, quantize, down; output norm, output, argmax x2 "weights_build_s": round(t_build, 1),
    }
    log(f"[bench] 8B decode: {out['tok_s']} tok/s ({us_tok:.1f} us/token, {out['gbs']} GB/s), "
        f"prompt positions {out['prompt_positions_tok_s']} tok/s")
    del dec, model
    torch.cuda.empty_cache()
    return out


def _timed_runs(fn, seconds, min_runs=5):
    fn()  # warm-up
    times = []
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds or len(times) < min_runs:
        a = time.perf_counter()
        fn()
        times.append(time.perf_counter() - a)
    times.sort()
    return times


def cpu_baseline(P, w_dev, x_dev, seconds):
    """ggml's CPU path restated with SIMD (oracle/cpu_ggml.cpp: Q8_0 activation and AVX-512 VNNI int8 block dots
    for the Q4_0 mat-vec; FP32-accumulating decode attention with F16C), timed on this host's cores on the same
    4096x14336 Q4_0 matrix and input as the roofline kernel, and FA decode at 8192 keys (32/8 heads, d 128); each
    the median of at least 5 runs over about seconds / 2."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import numpy as np

    import oracle

    oracle.build()
    w = w_dev.cpu().numpy()
    x = x_dev.cpu().numpy().reshape(1, -1)
    M, K = 4096, 14336
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or oracle.max_threads()
    # 32 copies of the matrix (1.06 GB), one per run in turn, so the host's last-level cache (up to a few hundred MB
    # on server parts) cannot hold the weights between runs.
    copies = [w.copy() for _ in range(32)]
    it = iter(range(1 << 60))
    mv = _timed_runs(lambda: oracle.cpu_mul_mat_q4_0(copies[next(it) % 32], M, K, x, nthreads=threads), seconds / 2)
    del copies
    med = mv[len(mv) // 2]
    b = matvec_bytes(P.Q4_0, M, K, 1)
    rng = np.random.default_rng(8192)
    q = rng.standard_normal(32 * 128).astype(np.float32)
    kv = [(rng.standard_normal(8 * 8192 * 128).astype(np.float16).view(np.uint16),
           rng.standard_normal(8 * 8192 * 128).astype(np.float16).view(np.uint16)) for _ in range(16)]  # 537 MB
    it2 = iter(range(1 << 60))

    def fa_run():
        k16, v16 = kv[next(it2) % 16]
        oracle.cpu_fa_decode(32, 8, 8192, 128, q, k16, v16, nthreads=threads)

    fa = _timed_runs(fa_run, seconds / 2)
    del kv
    fa_med = fa[len(fa) // 2]
    cpu = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    cpu = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    isa = "AVX-512 VNNI" if oracle.cpu_uses_vnni() else "AVX2"
    log(f"[bench] CPU q4_0 4096x14336 ({isa}): {med * 1e3:.3f} ms median of {len(mv)}; FA ctx 8192 "
        f"{fa_med * 1e6:.0f} us median of {len(fa)}; {threads} threads, {cpu}")
    return {"value": round(b / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"Q4_0 4096x14336 ne11=1 op (Q8_0 quantize of x + int8 block dots, ggml's CPU path restated "
                      f"with {isa}, OpenMP over rows) over 32 rotated copies of the matrix (1.06 GB): median "
                      f"{med * 1e3:.3f} ms of {len(mv)} runs (min {mv[0] * 1e3:.3f}, max {mv[-1] * 1e3:.3f}); {cpu}",
            "fa_decode_ctx8192": {"us": round(fa_med * 1e6, 1), "runs": len(fa),
                                  "gbs": round(fa_bytes(32, 8, 8192, 128) / fa_med / 1e9, 2),
                                  "note": "32/8 heads, d 128, fp16 K/V (16 rotated caches, 537 MB), FP32 online "
                                          "softmax per (head, KV chunk), chunks merged by log-sum-exp; F16C + FMA"}}


if __name__ == "__main__":
    main()
