"""Benchmark of the metalblas matmul hot path on one MI355X.

Headline (BASELINE.json ``metric``): bf16 GEMM 8192^3 in TFLOP/s and % of the dense bf16
MFMA peak.  One "step" is one C = A @ B of row-major 8192 x 8192 bf16 operands (synthetic
N(0,1) inputs from a fixed seed, resident in HBM before the timed region), i.e. one launch
of the matrix-core GEMM kernel.  The other BASELINE configurations are measured the same
way and reported under ``configs`` (GEMV 16384^2 in GB/s and % of HBM peak, the 2048 x 4096
x 2048 layouts and addmm, fp16 bmm / broadcast / split-K, complex64 GEMM and GEMV, int8
and int32 GEMM).  Prints ONE JSON line.

Timing: HIP events (torch.cuda.Event) on torch's current stream, which is the stream the
library launches its kernels on; W untimed warmup steps, then K timed steps bracketed by
device synchronisation.  ``roofline.traffic`` is the HBM bytes per launch measured with
rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by a plain-copy calibration); the figures
and the commands that produced them are in profiles/.

cpu_baseline: the CPU oracle (oracle/mb_oracle.c, a scalar restatement of the reference's
arithmetic) timed on whole output rows of the same 8192^3 workload for about --cpu-seconds;
cpu_torch: torch.matmul on all host cores over a row slab of the same workload, for context.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# MI355X published dense peaks
PEAK = {"bf16": 2516.6, "f16": 2516.6, "i8": 5033.2, "f32": 157.3}   # TFLOP/s (TOP/s for int8)
PEAK_HBM_GBS = 8000.0

# HBM bytes per launch from rocprofv3 --pmc (FETCH_SIZE x 2 + WRITE_SIZE x 1; the factors
# come from a 1 GiB copy, which reads as 512 MiB of FETCH_SIZE and 1 GiB of WRITE_SIZE):
# profiles/gemm_bf16_8192_pmc_traffic.md and profiles/gemv_bf16_16384_pmc_traffic.md
TRAFFIC = {
    "gemm_bf16_8192": 1.7823e9,
    "gemv_bf16_16384": 5.3745e8,
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--size", type=int, default=8192)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    p.add_argument("--only", choices=["all", "gemm", "gemv", "configs", "copy"], default="all",
                   help="gemm: the headline only; gemv: config 2 only; configs: every config but "
                        "the headline; copy: a plain 1 GiB device copy (HBM counter calibration)")
    p.add_argument("--no-tune", action="store_true", help="static plans only (the default)")
    p.add_argument("--tune", action="store_true", help="run the opt-in one-shot autotuner (METALBLAS_AUTOTUNE=1)")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    return p.parse_args()


# untimed GPU time before each secondary configuration's timed calls (the headline keeps the
# driver's W warmup steps: at 0.86 ms a call they already cover the clock ramp)
CFG_WARM_MS = 20.0
# timed calls of each secondary configuration, at least: the timed region starts from an idle,
# synchronised GPU, and that start costs about 100 us, which 20 calls of a 10 us product would
# read as 5 us a call (the headline times exactly the driver's K steps)
CFG_MIN_CALLS = 200


def time_events(torch, fn, steps, warmup, warm_ms=0.0):
    """ms per call of fn over `steps` calls (at least CFG_MIN_CALLS when warm_ms > 0), after
    `warmup` untimed calls and, when warm_ms > 0, more untimed calls until the GPU has run them
    for warm_ms (the clock ramps up over the first milliseconds of work after the host-side
    set-up, longer than 5 calls of a 50 us product)."""
    if warm_ms > 0:
        steps = max(steps, CFG_MIN_CALLS)
    for _ in range(warmup):
        fn()
    if warm_ms > 0:
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        while True:
            for _ in range(8):
                fn()
            e.record()
            e.synchronize()
            if s.elapsed_time(e) >= warm_ms:
                break
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def _gen(torch, seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------------------------------------
# headline: bf16 GEMM 8192^3
# ---------------------------------------------------------------------------------------------

def bench_headline(mb, torch, n, steps, warmup):
    g = _gen(torch, 0)
    a_cpu = torch.randn(n, n, generator=g).to(torch.bfloat16)
    b_cpu = torch.randn(n, n, generator=g).to(torch.bfloat16)
    a, b = a_cpu.cuda(), b_cpu.cuda()
    out = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")
    mb.matmul(a, b, out=out)            # planning (and the opt-in autotune) outside the timed region
    ms = time_events(torch, lambda: mb.matmul(a, b, out=out), steps, warmup)
    plan = mb.kernels.plan(a, b)
    return ms, plan, (a_cpu, b_cpu)


# ---------------------------------------------------------------------------------------------
# the other BASELINE configurations
# ---------------------------------------------------------------------------------------------

def _gemm_entry(name, ms, flops, peak_key, extra=None):
    tf = flops / (ms * 1e-3) / 1e12
    d = {"ms": round(ms, 5), "value": round(tf, 2), "unit": "TOP/s" if peak_key == "i8" else "TFLOP/s",
         "roofline": {"bound": "mfma", "peak": PEAK[peak_key], "frac": round(tf / PEAK[peak_key], 4)}}
    if extra:
        d.update(extra)
    return name, d


def _gemv_entry(name, ms, nbytes, extra=None):
    gbs = nbytes / (ms * 1e-3) / 1e9
    d = {"ms": round(ms, 5), "value": round(gbs, 1), "unit": "GB/s",
         "roofline": {"bound": "hbm", "peak": PEAK_HBM_GBS, "frac": round(gbs / PEAK_HBM_GBS, 4),
                      "algorithmic_bytes": int(nbytes)}}
    if extra:
        d.update(extra)
    return name, d


def bench_gemv(mb, torch, steps, warmup, n=16384):
    """Config 2: bf16 W 16384 x 16384 row-major; W@x (row streams), x@W (column streams),
    X(8 x K)@W (8 rows of x), W@X(K x 8)."""
    g = _gen(torch, 1)
    W = torch.randn(n, n, generator=g).to(torch.bfloat16).cuda()
    x = torch.randn(n, generator=g).to(torch.bfloat16).cuda()
    X8 = torch.randn(8, n, generator=g).to(torch.bfloat16).cuda()
    Xn = torch.randn(n, 8, generator=g).to(torch.bfloat16).cuda()
    res = {}
    y = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    ms = time_events(torch, lambda: mb.matmul(W, x, out=y), steps, warmup, CFG_WARM_MS)
    res.update([_gemv_entry("gemv_W@x", ms, 2.0 * (n * n + 2 * n), {"plan": mb.kernels.plan(W, x[:, None])["family"]})])
    ms = time_events(torch, lambda: mb.matmul(x, W, out=y), steps, warmup, CFG_WARM_MS)
    res.update([_gemv_entry("gemv_x@W", ms, 2.0 * (n * n + 2 * n), {"plan": mb.kernels.plan(x[None], W)["family"]})])
    Y8 = torch.empty(8, n, dtype=torch.bfloat16, device="cuda")
    ms = time_events(torch, lambda: mb.matmul(X8, W, out=Y8), steps, warmup, CFG_WARM_MS)
    res.update([_gemv_entry("gemv_X8@W", ms, 2.0 * (n * n + 16 * n))])
    Yn = torch.empty(n, 8, dtype=torch.bfloat16, device="cuda")
    ms = time_events(torch, lambda: mb.matmul(W, Xn, out=Yn), steps, warmup, CFG_WARM_MS)
    res.update([_gemv_entry("gemv_W@X8", ms, 2.0 * (n * n + 16 * n))])
    return res


def bench_layouts(mb, torch, steps, warmup, M=2048, K=4096, N=2048):
    """Config 3: bf16 2048 x 4096 @ 4096 x 2048 in every operand layout, plus addmm."""
    g = _gen(torch, 3)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = torch.randn(K, N, generator=g).to(torch.bfloat16)
    dev = "cuda"
    views = {
        "rm_rm": (A.cuda(), B.cuda()),
        "rm_cm": (A.cuda(), B.t().contiguous().cuda().t()),
        "cm_rm": (A.t().contiguous().cuda().t(), B.cuda()),
        "cm_cm": (A.t().contiguous().cuda().t(), B.t().contiguous().cuda().t()),
        "row_sliced": (torch.randn(2 * M, K, generator=g).to(torch.bfloat16).cuda()[::2], B.cuda()),
        "col_sliced": (torch.randn(M, 2 * K, generator=g).to(torch.bfloat16).cuda()[:, ::2], B.cuda()),
        "offset17": (torch.cat([torch.zeros(17, dtype=torch.bfloat16), A.reshape(-1)]).cuda()[17:].view(M, K),
                     B.cuda()),
    }
    flops = 2.0 * M * N * K
    res = {}
    out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    for name, (a, b) in views.items():
        ms = time_events(torch, lambda: mb.matmul(a, b, out=out), steps, warmup, CFG_WARM_MS)
        res.update([_gemm_entry(f"bf16_2048x4096x2048_{name}", ms, flops, "bf16",
                                {"plan": mb.kernels.plan(a if name != "col_sliced" else a.contiguous(), b)["family"]})])
    bias = torch.randn(N, generator=g).to(torch.bfloat16).cuda()
    a, b = views["rm_rm"]
    ms = time_events(torch, lambda: mb.addmm(bias, a, b, beta=0.5, alpha=2.0, out=out), steps, warmup, CFG_WARM_MS)
    res.update([_gemm_entry("bf16_2048x4096x2048_addmm", ms, flops, "bf16")])
    return res


def bench_bmm(mb, torch, steps, warmup):
    """Config 4: fp16 bmm 8 x (512x256 @ 256x512), broadcast B, split-K 1 x 128 x 65536."""
    g = _gen(torch, 4)
    a = torch.randn(8, 512, 256, generator=g).to(torch.float16).cuda()
    b = torch.randn(8, 256, 512, generator=g).to(torch.float16).cuda()
    b2 = torch.randn(256, 512, generator=g).to(torch.float16).cuda()
    res = {}
    fl = 2.0 * 8 * 512 * 512 * 256
    ms = time_events(torch, lambda: mb.bmm(a, b), steps, warmup, CFG_WARM_MS)
    res.update([_gemm_entry("f16_bmm_8x512x512x256", ms, fl, "f16")])
    ms = time_events(torch, lambda: mb.matmul(a, b2), steps, warmup, CFG_WARM_MS)
    res.update([_gemm_entry("f16_bmm_broadcastB", ms, fl, "f16")])
    ak = torch.randn(1, 128, 65536, generator=g).to(torch.float16).cuda()
    bk = torch.randn(1, 65536, 128, generator=g).to(torch.float16).cuda()
    ms = time_events(torch, lambda: mb.bmm(ak, bk), steps, warmup, CFG_WARM_MS)
    nbytes = 2.0 * (2 * 128 * 65536 + 128 * 128)
    name, d = _gemm_entry("f16_splitk_128x128x65536", ms, 2.0 * 128 * 128 * 65536, "f16")
    gbs = nbytes / (ms * 1e-3) / 1e9
    d["hbm"] = {"value": round(gbs, 1), "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                "note": "arithmetic intensity 64 flop/B: HBM-bound"}
    res[name] = d
    return res


def bench_mixed(mb, torch, steps, warmup):
    """Config 5: complex64 GEMM 2048^3 with conj(A), complex64 GEMV 8192^2, int8 GEMM 4096^3;
    config 1: int32 GEMM 256^3."""
    g = _gen(torch, 5)
    res = {}
    n = 2048
    a = torch.complex(torch.randn(n, n, generator=g), torch.randn(n, n, generator=g)).cuda()
    b = torch.complex(torch.randn(n, n, generator=g), torch.randn(n, n, generator=g)).cuda()
    ms = time_events(torch, lambda: mb.matmul(a.conj(), b), steps, warmup, CFG_WARM_MS)
    res.update([_gemm_entry("c64_gemm_2048_conjA", ms, 8.0 * n ** 3, "f32",
                            {"plan": mb.kernels.plan(a, b)["family"]})])
    m = 8192
    A = torch.complex(torch.randn(m, m, generator=g), torch.randn(m, m, generator=g)).cuda()
    x = torch.complex(torch.randn(m, generator=g), torch.randn(m, generator=g)).cuda()
    ms = time_events(torch, lambda: mb.matmul(A, x), steps, warmup, CFG_WARM_MS)
    res.update([_gemv_entry("c64_gemv_8192", ms, 8.0 * (m * m + 2 * m))])
    del A, x
    k = 4096
    ai = torch.randint(-4, 5, (k, k), generator=g, dtype=torch.int8).cuda()
    bi = torch.randint(-4, 5, (k, k), generator=g, dtype=torch.int8).cuda()
    ms = time_events(torch, lambda: mb.matmul(ai, bi), steps, warmup, CFG_WARM_MS)
    res.update([_gemm_entry("i8_gemm_4096", ms, 2.0 * k ** 3, "i8", {"plan": mb.kernels.plan(ai, bi)["family"]})])
    s = 256
    a32 = torch.randint(-8, 9, (s, s), generator=g, dtype=torch.int32).cuda()
    b32 = torch.randint(-8, 9, (s, s), generator=g, dtype=torch.int32).cuda()
    ms = time_events(torch, lambda: mb.matmul(a32, b32), steps, warmup, CFG_WARM_MS)
    res["i32_gemm_256"] = {"ms": round(ms, 5), "us": round(ms * 1e3, 2),
                           "value": round(2.0 * s ** 3 / (ms * 1e-3) / 1e9, 1), "unit": "GOP/s",
                           "roofline": {"bound": "launch", "note": "33.6 M int-ops: launch/latency bound"},
                           "plan": mb.kernels.plan(a32, b32)["family"]}
    return res


# ---------------------------------------------------------------------------------------------
# CPU baselines
# ---------------------------------------------------------------------------------------------

def cpu_oracle_gemm(a_cpu, b_cpu, seconds):
    """The scalar oracle on whole output rows of the workload until ~seconds have elapsed."""
    import oracle
    n = a_cpu.shape[0]
    rows_done, r = 0, 0
    t0 = time.perf_counter()
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
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    rows = 256
    a = a_cpu[:rows]
    torch.matmul(a, b_cpu)
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
        print(json.dumps({"error": "this build measures one GPU: run with --gpus 1 (the multi-GPU "
                          "sharding of the path is a design, not a measured configuration)"}))
        sys.exit(2)
    if args.tune and not args.no_tune:
        os.environ["METALBLAS_AUTOTUNE"] = "1"
    else:
        os.environ["METALBLAS_AUTOTUNE"] = "0"
    import torch
    import metalblas_amd as mb

    if args.only == "copy":
        nbytes = 1 << 30
        src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        ms = time_events(torch, lambda: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"copy_bytes_each_way": nbytes, "ms": round(ms, 4),
                          "GBps_read_plus_write": round(2 * nbytes / ms / 1e6, 1)}))
        return

    n = args.size
    result = {
        "metric": "TFLOP/s + % MFMA peak (bf16 GEMM 8192³); GEMV HBM GB/s + % peak",
        "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) inputs from torch.Generator seeds, resident in HBM",
        "config": {"workload": f"bf16 GEMM C = A @ B, {n} x {n} x {n}, row-major A and B "
                               "(BASELINE config 3, square case)", "parallelism": "single GPU"},
    }
    headline = None
    if args.only in ("all", "gemm"):
        ms, plan, headline = bench_headline(mb, torch, n, args.steps, args.warmup)
        flops = 2.0 * n ** 3
        tf = flops / (ms * 1e-3) / 1e12
        result["value"] = round(tf, 2)
        result["ms_per_step"] = round(ms, 4)
        result["roofline"] = {
            "bound": "mfma", "achieved": round(tf, 2), "peak": PEAK["bf16"], "unit": "TFLOP/s",
            "frac": round(tf / PEAK["bf16"], 4),
            "traffic": TRAFFIC["gemm_bf16_8192"] if n == 8192 else None,
            "kernel": f"matrix-core GEMM tile {plan['tile'][0]}x{plan['tile'][1]} "
                      f"schedule {'ping-pong' if plan['tile'][5] == 2 else 'interleaved'}",
            "algorithmic_per_launch": f"2*{n}^3 = {flops:.4e} flop",
            "avg_launch_ms": round(ms, 4),
        }
        result["plan"] = {k: plan[k] for k in ("family", "tile", "split_k", "grid")}
    if args.only in ("all", "gemv", "configs"):
        cfg = {}
        cfg.update(bench_gemv(mb, torch, args.steps, args.warmup))
        if args.only != "gemv":
            cfg.update(bench_layouts(mb, torch, args.steps, args.warmup))
            cfg.update(bench_bmm(mb, torch, args.steps, args.warmup))
            cfg.update(bench_mixed(mb, torch, args.steps, args.warmup))
        g = cfg["gemv_W@x"]
        g["roofline"]["traffic"] = TRAFFIC["gemv_bf16_16384"]
        result["configs"] = cfg
        result["configs_timing"] = (f"each config: {args.warmup} warmup calls, {CFG_WARM_MS:g} ms of untimed "
                                    f"calls, then {max(args.steps, CFG_MIN_CALLS)} timed calls (HIP events)")
        if result["value"] is None:
            result.update({"value": g["value"], "unit": "GB/s", "ms_per_step": g["ms"],
                           "roofline": dict(g["roofline"], achieved=g["value"], unit="GB/s")})
    if not args.no_cpu and headline is not None:
        a_cpu, b_cpu = headline
        v, rows, el = cpu_oracle_gemm(a_cpu, b_cpu, args.cpu_seconds)
        result["cpu_baseline"] = {
            "value": round(v, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"oracle/mb_oracle.c (scalar fp64 restatement) on {rows} whole output rows of the "
                      f"{n}^3 bf16 GEMM, {el:.1f} s",
        }
        v2, rows2, it2, thr = cpu_torch_gemm(torch, a_cpu, b_cpu, max(2.0, args.cpu_seconds / 2))
        result["cpu_torch"] = {"value": round(v2, 4), "unit": "TFLOP/s", "cores": thr,
                               "kind": "torch.matmul bf16 on the host CPU",
                               "sample": f"{rows2} x {n} x {n} slab x {it2}"}
    print(json.dumps(result))


if __name__ == "__main__":
    main()
