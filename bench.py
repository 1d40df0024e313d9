"""Benchmark of the metalblas matmul hot path on one MI355X.

Headline (BASELINE.json metric): bf16 GEMM 8192^3 in TFLOP/s and % of the dense bf16 MFMA
peak, plus bf16 GEMV 16384x16384 (y = W @ x) in GB/s and % of HBM peak.  One "step" is one
8192^3 product C = A @ B (row-major A and B, synthetic N(0,1) inputs from a fixed seed,
already resident in HBM).  Prints ONE JSON line.

Timing: HIP events on torch's current stream, which is the stream the library launches on.
cpu_baseline: the CPU oracle (oracle/mb_oracle.c, a scalar port of the reference semantics)
timed on a bounded sample of the same workload (a few output rows); cpu_torch: torch.matmul
on the host cores for context (north star).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6     # 256 CU x 4096 flop/clk x 2.4 GHz (dense)
PEAK_HBM_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--size", type=int, default=8192)
    p.add_argument("--gemv", type=int, default=16384)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    p.add_argument("--only", choices=["all", "gemm", "gemv", "copy"], default="all",
                   help="copy: a plain 1 GiB device copy, the calibration run for HBM counters")
    p.add_argument("--no-tune", action="store_true", help="static plans only (METALBLAS_AUTOTUNE=0)")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


def time_events(fn, steps):
    import torch
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps   # ms per call


def bench_gemm(mb, torch, n, steps, warmup):
    g = torch.Generator().manual_seed(0)
    a_cpu = torch.randn(n, n, generator=g).to(torch.bfloat16)
    b_cpu = torch.randn(n, n, generator=g).to(torch.bfloat16)
    a, b = a_cpu.cuda(), b_cpu.cuda()
    out = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")
    for _ in range(warmup):
        mb.matmul(a, b, out=out)
    torch.cuda.synchronize()
    ms = time_events(lambda: mb.matmul(a, b, out=out), steps)
    plan = mb.kernels.plan(a, b)
    return ms, plan, (a_cpu, b_cpu, out)


def bench_gemv(mb, torch, n, steps, warmup):
    g = torch.Generator().manual_seed(1)
    W_cpu = torch.randn(n, n, generator=g).to(torch.bfloat16)
    x_cpu = torch.randn(n, generator=g).to(torch.bfloat16)
    W, x = W_cpu.cuda(), x_cpu.cuda()
    y = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    for _ in range(warmup):
        mb.matmul(W, x, out=y)
    ms = time_events(lambda: mb.matmul(W, x, out=y), steps)
    # x @ W (the column-streaming family) moves the same bytes
    yt = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    for _ in range(warmup):
        mb.matmul(x, W, out=yt)
    ms_t = time_events(lambda: mb.matmul(x, W, out=yt), steps)
    plan = mb.kernels.plan(W, x.reshape(-1, 1))
    return ms, ms_t, plan, (W_cpu, x_cpu, y)


def cpu_oracle_gemm(a_cpu, b_cpu, seconds):
    """Time the scalar oracle on whole output rows until ~seconds have elapsed."""
    import oracle
    n = a_cpu.shape[0]
    rows_done = 0
    t0 = time.perf_counter()
    r = 0
    while True:
        oracle.gemm(a_cpu, b_cpu, rows=[r])
        rows_done += 1
        r = (r + 977) % n
        el = time.perf_counter() - t0
        if el >= seconds or rows_done >= n:
            break
    flops = 2.0 * rows_done * b_cpu.shape[1] * a_cpu.shape[1]
    return flops / el / 1e12, rows_done, el


def cpu_torch_gemm(torch, a_cpu, b_cpu, seconds):
    """torch.matmul on the host cores over a row slab of the same workload."""
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    rows = 256
    a = a_cpu[:rows]
    torch.matmul(a, b_cpu)   # warmup
    t0 = time.perf_counter()
    it = 0
    while True:
        torch.matmul(a, b_cpu)
        it += 1
        el = time.perf_counter() - t0
        if el >= seconds or it >= 50:
            break
    flops = 2.0 * rows * b_cpu.shape[1] * a_cpu.shape[1] * it
    return flops / el / 1e12, rows, it, threads


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only (--gpus 1); the multi-GPU "
                          "sharding is a design in DESIGN.md, not a measured path"}))
        sys.exit(2)
    if args.no_tune:
        os.environ["METALBLAS_AUTOTUNE"] = "0"
    import torch
    import metalblas_amd as mb
    if args.only == "copy":
        nbytes = 1 << 30
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(args.warmup):
            dst.copy_(src)
        ms = time_events(lambda: dst.copy_(src), args.steps)
        print(json.dumps({"copy_bytes_each_way": nbytes, "ms": round(ms, 4),
                          "GBps_read_plus_write": round(2 * nbytes / ms / 1e6, 1)}))
        return

    result = {
        "metric": "TFLOP/s + % MFMA peak (bf16 GEMM 8192³); GEMV HBM GB/s + % peak",
        "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 inputs from torch.Generator seed 0, resident in HBM",
        "config": {"workload": f"bf16 GEMM C=A@B {args.size}x{args.size}x{args.size}, row-major A and B "
                               "(BASELINE config 3, square case)",
                   "gemv_workload": f"bf16 GEMV y=W@x W {args.gemv}x{args.gemv} row-major (config 2)",
                   "parallelism": "single GPU"},
    }
    gemm_data = gemv_data = None
    if args.only in ("all", "gemm"):
        n = args.size
        ms, plan, gemm_data = bench_gemm(mb, torch, n, args.steps, args.warmup)
        flops = 2.0 * n * n * n
        tflops = flops / (ms * 1e-3) / 1e12
        result["value"] = round(tflops, 2)
        result["ms_per_step"] = round(ms, 4)
        result["roofline"] = {
            "bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": None,
            "kernel": f"k_gemm_mfma<bf16,{plan['tile'][0]},{plan['tile'][1]}>",
            "algorithmic_per_launch": f"2*{n}^3 = {flops:.4e} flop",
            "avg_launch_ms": round(ms, 4),
        }
        result["plan"] = {k: plan[k] for k in ("family", "tile", "split_k", "grid")}
    if args.only in ("all", "gemv"):
        n = args.gemv
        ms, ms_t, plan, gemv_data = bench_gemv(mb, torch, n, args.steps, args.warmup)
        nbytes = 2.0 * (n * n + n + n)
        gbs = nbytes / (ms * 1e-3) / 1e9
        gbs_t = nbytes / (ms_t * 1e-3) / 1e9
        result["gemv"] = {
            "value": round(gbs, 1), "unit": "GB/s", "ms": round(ms, 4),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                         "algorithmic_per_launch": f"2*({n}^2+2*{n}) = {nbytes:.4e} B"},
            "x_at_W": {"value": round(gbs_t, 1), "unit": "GB/s", "ms": round(ms_t, 4),
                       "frac": round(gbs_t / PEAK_HBM_GBS, 4)},
            "plan": plan["family"],
        }
        if result["value"] is None:
            result.update({"value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(ms, 4)})
    if not args.no_cpu and gemm_data is not None:
        a_cpu, b_cpu, _ = gemm_data
        v, rows, el = cpu_oracle_gemm(a_cpu, b_cpu, args.cpu_seconds)
        result["cpu_baseline"] = {
            "value": round(v, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"oracle/mb_oracle.c (scalar fp64 restatement) on {rows} output rows of the "
                      f"{args.size}^3 bf16 GEMM, {el:.1f} s",
        }
        v2, rows2, it2, thr = cpu_torch_gemm(torch, a_cpu, b_cpu, max(2.0, args.cpu_seconds / 2))
        result["cpu_torch"] = {
            "value": round(v2, 4), "unit": "TFLOP/s", "cores": thr, "kind": "torch.matmul bf16 CPU",
            "sample": f"{rows2}x{args.size}x{args.size} slab x{it2}",
        }
    print(json.dumps(result))


if __name__ == "__main__":
    main()
