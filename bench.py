"""Benchmark of the metalblas matmul hot path on one MI355X.

Headline (BASELINE.json ``metric``): bf16 GEMM 8192^3 in TFLOP/s and % of the dense bf16
MFMA peak.  One "step" is one C = A @ B of row-major 8192 x 8192 bf16 operands (synthetic
N(0,1) inputs from a fixed seed, resident in HBM before the timed region), i.e. one launch
of the matrix-core GEMM kernel.  The other BASELINE configurations are measured the same
way and reported under ``configs`` (GEMV 16384^2 in GB/s and % of HBM peak, the 2048 x 4096
x 2048 layouts and addmm, fp16 bmm / broadcast / split-K, complex64 GEMM and GEMV, int8
and int32 GEMM).  Prints ONE JSON line.

Every timed call is one entry of ``WORKLOADS`` below; tests/test_gpu_configs.py builds the same
entries and checks each one's output against the CPU oracle, so no number here rests on an
output that no test compared.

Timing: HIP events (torch.cuda.Event) on torch's current stream, which is the stream the
library launches its kernels on; W untimed warmup steps, then K timed steps bracketed by
device synchronisation.  ``roofline.traffic`` is the HBM bytes per launch measured with
rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by a plain-copy calibration); the figures
and the commands that produced them are in profiles/.

cpu_baseline: torch.matmul / addmm / bmm on the host CPU (the baseline BASELINE.json names:
the reference's kernels are Metal-only), on the same seeded CPU tensors that were copied to the
GPU, with the thread count and CPU model recorded; 1 warmup, then at least 3 timed runs and at
least 1 s, best run reported.  The headline and the int8 product are timed on a row slab of the
workload (stated in ``sample``); every other config on the whole workload.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# MI355X published dense peaks
PEAK = {"bf16": 2516.6, "f16": 2516.6, "i8": 5033.2, "f32": 157.3}   # TFLOP/s (TOP/s for int8)
PEAK_HBM_GBS = 8000.0

# HBM-side bytes per launch of each workload's dominant kernel over its timed calls: rocprofv3
# FETCH_SIZE x 2 + WRITE_SIZE (KiB x 1024; the factors come from a 1 GiB device copy), from
# profiles/gemm_bf16_8192_counters.md and profiles/configs_counters.md
TRAFFIC = {
    "bf16_gemm_8192": 1.7862e+09,                   # k_gemm16pp<bf16, ...>
    "gemv_W@x": 5.3746e+08,                         # k_dot_wg
    "gemv_x@W": 5.4544e+08,                         # k_axpy_band (+ its fp32 planes)
    "gemv_Wt@x": 5.4544e+08,                        # k_axpy_band, as x@W
    "gemv_X8@W": 5.4012e+08,                        # k_thin16 32 x 128
    "gemv_W@X8": 5.3933e+08,                        # k_dotx
    "bf16_2048x4096x2048_rm_rm": 1.0938e+08,        # k_gemm16 128 x 128
    "bf16_2048x4096x2048_rm_cm": 1.0938e+08,
    "bf16_2048x4096x2048_cm_rm": 1.0939e+08,
    "bf16_2048x4096x2048_cm_cm": 1.0938e+08,
    "bf16_2048x4096x2048_row_sliced": 1.0938e+08,
    "bf16_2048x4096x2048_col_sliced": 1.0938e+08,
    "bf16_2048x4096x2048_offset17": 1.0938e+08,
    "bf16_2048x4096x2048_addmm": 1.0941e+08,
    "f16_bmm_8x512x512x256": 2.3314e+07,            # k_gemm16 (the tile the tuner took: 128 x 64)
    "f16_bmm_broadcastB": 9.6800e+06,               # k_gemm16 128 x 64
    "f16_splitk_128x128x65536": 3.7852e+07,         # the deep-K k_thin16 64 x 64
    "c64_gemm_2048_conjA": 3.7610e+08,              # k_gemm_mfma<float> after k_cplx_expand
    "c64_gemv_8192": 5.3758e+08,                    # k_cdot_wg
    "i8_gemm_4096": 1.1798e+08,                     # k_gemm16pp<int8, ...>
    "i32_gemm_256": 2.9991e+06,                     # k_gemm_generic<int32, 16>
}


def parse(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--size", type=int, default=8192)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    p.add_argument("--only", default="all",
                   help="all | gemm (the headline only) | configs (every config but the headline) | "
                        "copy (a plain 1 GiB device copy: HBM counter calibration) | a comma-separated "
                        "list of workload groups (headline, gemv, layouts, bmm, c64, int) or names")
    p.add_argument("--no-tune", action="store_true",
                   help="static plans only (METALBLAS_AUTOTUNE=0); the default is the library's "
                        "one-shot autotuner, as in the reference")
    p.add_argument("--calls", type=int, default=0,
                   help="timed calls of each secondary configuration (default: at least 200); for "
                        "profiling runs, where every dispatch is collected")
    p.add_argument("--cpu-threads", type=int, default=0,
                   help="threads for the CPU baseline (default: OMP_NUM_THREADS, else all cores)")
    return p.parse_args(argv)


# untimed GPU time before each secondary configuration's timed calls (the headline keeps the
# driver's W warmup steps: at 0.86 ms a call they already cover the clock ramp)
CFG_WARM_MS = 20.0
# timed calls of each secondary configuration, at least: the timed region starts from an idle,
# synchronised GPU, and that start costs about 100 us, which 20 calls of a 10 us product would
# read as 5 us a call (the headline times exactly the driver's K steps)
CFG_MIN_CALLS = 200


def time_events(torch, fn, steps, warmup, warm_ms=0.0, calls=0):
    """ms per call of fn over `steps` calls (when warm_ms > 0: `calls` calls if given, else at
    least CFG_MIN_CALLS), after `warmup` untimed calls and, when warm_ms > 0, more untimed calls
    until the GPU has run them for warm_ms (the clock ramps up over the first milliseconds of
    work after the host-side set-up, longer than 5 calls of a 50 us product)."""
    if warm_ms > 0:
        steps = calls if calls > 0 else max(steps, CFG_MIN_CALLS)
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


# ---------------------------------------------------------------------------------------------
# the BASELINE workloads
# ---------------------------------------------------------------------------------------------

class Workload:
    """One timed call and everything needed to check and price it.

    call()       queues the product on the GPU and returns its output tensor;
    check        (view, a, b, kwargs): ``view(out)`` is the output as a 2-D / 3-D product of the
                 device operands ``a`` @ ``b`` (views in the benched layout), kwargs the epilogue
                 (bias / beta / alpha) -- what the parity test compares with the oracle;
    flops/nbytes the algorithmic work of one call; ``bound`` says which one prices it;
    cpu()        the same operation with torch on the host CPU, over ``cpu_frac`` of the workload.
    """

    def __init__(self, name, cfg, call, check, *, flops, nbytes, bound, peak_key=None, cpu=None,
                 cpu_frac=1.0, cpu_sample="the whole workload", note=None):
        self.name, self.cfg, self.call, self.check = name, cfg, call, check
        self.flops, self.nbytes, self.bound, self.peak_key = flops, nbytes, bound, peak_key
        self.cpu, self.cpu_frac, self.cpu_sample, self.note = cpu, cpu_frac, cpu_sample, note


def _gen(torch, seed):
    return torch.Generator().manual_seed(seed)


def _plain(out):
    return out


def group_headline(torch, mb, n=8192):
    """Config 3, square case: bf16 8192^3, row-major A and B, seed 0."""
    g = _gen(torch, 0)
    a_cpu = torch.randn(n, n, generator=g).to(torch.bfloat16)
    b_cpu = torch.randn(n, n, generator=g).to(torch.bfloat16)
    a, b = a_cpu.cuda(), b_cpu.cuda()
    out = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")
    slab = max(1, n // 8)
    return [Workload(f"bf16_gemm_{n}", "3", lambda: mb.matmul(a, b, out=out), (_plain, a, b, {}),
                     flops=2.0 * n ** 3, nbytes=2.0 * 3 * n * n, bound="mfma", peak_key="bf16",
                     cpu=lambda: torch.matmul(a_cpu[:slab], b_cpu), cpu_frac=slab / n,
                     cpu_sample=f"{slab} x {n} x {n} row slab ({slab} of the {n} output rows)")]


def group_gemv(torch, mb, n=16384):
    """Config 2: bf16 W 16384 x 16384 row-major; W@x (the reference's gemv_nt), x@W (gemv_t),
    W^T@x (the transposed-W case), X(8 x K)@W (8 rows of x), W@X(K x 8)."""
    g = _gen(torch, 1)
    Wc = torch.randn(n, n, generator=g).to(torch.bfloat16)
    xc = torch.randn(n, generator=g).to(torch.bfloat16)
    X8c = torch.randn(8, n, generator=g).to(torch.bfloat16)
    Xnc = torch.randn(n, 8, generator=g).to(torch.bfloat16)
    W, x, X8, Xn = Wc.cuda(), xc.cuda(), X8c.cuda(), Xnc.cuda()
    y = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    y3 = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    Y8 = torch.empty(8, n, dtype=torch.bfloat16, device="cuda")
    Yn = torch.empty(n, 8, dtype=torch.bfloat16, device="cuda")
    one = 2.0 * (n * n + 2 * n)
    eight = 2.0 * (n * n + 16 * n)
    return [
        Workload("gemv_W@x", "2", lambda: mb.matmul(W, x, out=y),
                 (lambda o: o.reshape(n, 1), W, x.reshape(n, 1), {}),
                 flops=2.0 * n * n, nbytes=one, bound="hbm", cpu=lambda: torch.matmul(Wc, xc)),
        Workload("gemv_x@W", "2", lambda: mb.matmul(x, W, out=y2),
                 (lambda o: o.reshape(1, n), x.reshape(1, n), W, {}),
                 flops=2.0 * n * n, nbytes=one, bound="hbm", cpu=lambda: torch.matmul(xc, Wc)),
        # W^T @ x on the same row-major W (BASELINE's "transposed-W" variant): the matrix is
        # read down its columns, so it streams like x @ W
        Workload("gemv_Wt@x", "2", lambda: mb.matmul(W.t(), x, out=y3),
                 (lambda o: o.reshape(n, 1), W.t(), x.reshape(n, 1), {}),
                 flops=2.0 * n * n, nbytes=one, bound="hbm", cpu=lambda: torch.matmul(Wc.t(), xc)),
        Workload("gemv_X8@W", "2", lambda: mb.matmul(X8, W, out=Y8), (_plain, X8, W, {}),
                 flops=16.0 * n * n, nbytes=eight, bound="hbm", cpu=lambda: torch.matmul(X8c, Wc)),
        Workload("gemv_W@X8", "2", lambda: mb.matmul(W, Xn, out=Yn), (_plain, W, Xn, {}),
                 flops=16.0 * n * n, nbytes=eight, bound="hbm", cpu=lambda: torch.matmul(Wc, Xnc)),
    ]


def layout_views(torch, M=2048, K=4096, N=2048, seed=3):
    """Config 3 operands: bf16 A 2048 x 4096 and B 4096 x 2048 ~ N(0,1) in every layout the
    BASELINE names, as (CPU view, GPU view) pairs of the same layout, plus the addmm bias."""
    g = _gen(torch, seed)
    A = torch.randn(M, K, generator=g).to(torch.bfloat16)
    B = torch.randn(K, N, generator=g).to(torch.bfloat16)
    Acm = A.t().contiguous().t()
    Bcm = B.t().contiguous().t()
    Arow = torch.randn(2 * M, K, generator=g).to(torch.bfloat16)
    Acol = torch.randn(M, 2 * K, generator=g).to(torch.bfloat16)
    Aoff = torch.cat([torch.zeros(17, dtype=torch.bfloat16), A.reshape(-1)])
    bias = torch.randn(N, generator=g).to(torch.bfloat16)

    def cm(t):   # a column-major device copy of a column-major CPU view
        return t.t().contiguous().cuda().t()
    Ad, Bd = A.cuda(), B.cuda()
    views = {
        "rm_rm": ((A, B), (Ad, Bd)),
        "rm_cm": ((A, Bcm), (Ad, cm(Bcm))),
        "cm_rm": ((Acm, B), (cm(Acm), Bd)),
        "cm_cm": ((Acm, Bcm), (cm(Acm), cm(Bcm))),
        # every other row of a 2x taller buffer (the reference benchmark's "sliced")
        "row_sliced": ((Arow[::2], B), (Arow.cuda()[::2], Bd)),
        # every other column of a 2x wider buffer (BASELINE's "sliced"; copied, as the reference does)
        "col_sliced": ((Acol[:, ::2], B), (Acol.cuda()[:, ::2], Bd)),
        # a contiguous view at storage offset 17 elements
        "offset17": ((Aoff[17:].view(M, K), B), (Aoff.cuda()[17:].view(M, K), Bd)),
    }
    return views, (bias, bias.cuda())


def group_layouts(torch, mb, M=2048, K=4096, N=2048):
    """Config 3: bf16 2048 x 4096 @ 4096 x 2048 in every operand layout, plus addmm
    (bias of length 2048, beta 0.5, alpha 2)."""
    views, (bias_c, bias) = layout_views(torch, M, K, N)
    out = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    flops = 2.0 * M * N * K
    nbytes = 2.0 * (M * K + K * N + M * N)
    res = []
    for name, ((ac, bc), (a, b)) in views.items():
        res.append(Workload(f"bf16_2048x4096x2048_{name}", "3",
                            (lambda a=a, b=b: mb.matmul(a, b, out=out)), (_plain, a, b, {}),
                            flops=flops, nbytes=nbytes, bound="mfma", peak_key="bf16",
                            cpu=(lambda ac=ac, bc=bc: torch.matmul(ac, bc))))
    (ac, bc), (a, b) = views["rm_rm"]
    res.append(Workload("bf16_2048x4096x2048_addmm", "3",
                        lambda: mb.addmm(bias, a, b, beta=0.5, alpha=2.0, out=out),
                        (_plain, a, b, {"bias": bias, "beta": 0.5, "alpha": 2.0}),
                        flops=flops, nbytes=nbytes + 2.0 * N, bound="mfma", peak_key="bf16",
                        cpu=lambda: torch.addmm(bias_c, ac, bc, beta=0.5, alpha=2.0)))
    return res


def group_bmm(torch, mb):
    """Config 4: fp16 bmm 8 x (512x256 @ 256x512), A 8x512x256 @ shared B 256x512, and split-K
    1 x 128 x 65536 @ 1 x 65536 x 128."""
    g = _gen(torch, 4)
    ac = torch.randn(8, 512, 256, generator=g).to(torch.float16)
    bc = torch.randn(8, 256, 512, generator=g).to(torch.float16)
    b2c = torch.randn(256, 512, generator=g).to(torch.float16)
    akc = torch.randn(1, 128, 65536, generator=g).to(torch.float16)
    bkc = torch.randn(1, 65536, 128, generator=g).to(torch.float16)
    a, b, b2, ak, bk = ac.cuda(), bc.cuda(), b2c.cuda(), akc.cuda(), bkc.cuda()
    fl = 2.0 * 8 * 512 * 512 * 256
    return [
        Workload("f16_bmm_8x512x512x256", "4", lambda: mb.bmm(a, b), (_plain, a, b, {}),
                 flops=fl, nbytes=2.0 * 8 * (512 * 256 * 2 + 512 * 512), bound="mfma", peak_key="f16",
                 cpu=lambda: torch.bmm(ac, bc)),
        Workload("f16_bmm_broadcastB", "4", lambda: mb.matmul(a, b2),
                 (_plain, a, b2.expand(8, 256, 512), {}),
                 flops=fl, nbytes=2.0 * (8 * 512 * 256 + 256 * 512 + 8 * 512 * 512), bound="mfma",
                 peak_key="f16", cpu=lambda: torch.matmul(ac, b2c)),
        Workload("f16_splitk_128x128x65536", "4", lambda: mb.bmm(ak, bk), (_plain, ak, bk, {}),
                 flops=2.0 * 128 * 128 * 65536, nbytes=2.0 * (2 * 128 * 65536 + 128 * 128),
                 bound="hbm", peak_key="f16", cpu=lambda: torch.bmm(akc, bkc),
                 note="arithmetic intensity 64 flop/B, under the ridge: HBM-bound"),
    ]


def group_c64(torch, mb):
    """Config 5a/5b: complex64 GEMM 2048^3 with conj(A), complex64 GEMV 8192^2."""
    g = _gen(torch, 5)
    n = 2048
    ac = torch.complex(torch.randn(n, n, generator=g), torch.randn(n, n, generator=g))
    bc = torch.complex(torch.randn(n, n, generator=g), torch.randn(n, n, generator=g))
    a, b = ac.cuda(), bc.cuda()
    out = torch.empty(n, n, dtype=torch.complex64, device="cuda")
    m = 8192
    Ac = torch.complex(torch.randn(m, m, generator=g), torch.randn(m, m, generator=g))
    xc = torch.complex(torch.randn(m, generator=g), torch.randn(m, generator=g))
    A, x = Ac.cuda(), xc.cuda()
    y = torch.empty(m, dtype=torch.complex64, device="cuda")
    return [
        Workload("c64_gemm_2048_conjA", "5a", lambda: mb.matmul(a.conj(), b, out=out),
                 (_plain, a.conj(), b, {}), flops=8.0 * n ** 3, nbytes=8.0 * 3 * n * n, bound="mfma",
                 peak_key="f32", cpu=lambda: torch.matmul(ac.conj(), bc)),
        Workload("c64_gemv_8192", "5b", lambda: mb.matmul(A, x, out=y),
                 (lambda o: o.reshape(m, 1), A, x.reshape(m, 1), {}),
                 flops=8.0 * m * m, nbytes=8.0 * (m * m + 2 * m), bound="hbm",
                 cpu=lambda: torch.matmul(Ac, xc)),
    ]


def group_int(torch, mb):
    """Config 5c: int8 4096^3 in [-4, 4]; config 1: int32 256^3 in [-8, 8]."""
    g = _gen(torch, 6)
    k = 4096
    aic = torch.randint(-4, 5, (k, k), generator=g, dtype=torch.int8)
    bic = torch.randint(-4, 5, (k, k), generator=g, dtype=torch.int8)
    ai, bi = aic.cuda(), bic.cuda()
    oi = torch.empty(k, k, dtype=torch.int8, device="cuda")
    s = 256
    a32c = torch.randint(-8, 9, (s, s), generator=g, dtype=torch.int32)
    b32c = torch.randint(-8, 9, (s, s), generator=g, dtype=torch.int32)
    a32, b32 = a32c.cuda(), b32c.cuda()
    o32 = torch.empty(s, s, dtype=torch.int32, device="cuda")
    slab = 256
    return [
        Workload("i8_gemm_4096", "5c", lambda: mb.matmul(ai, bi, out=oi), (_plain, ai, bi, {}),
                 flops=2.0 * k ** 3, nbytes=3.0 * k * k, bound="mfma", peak_key="i8",
                 cpu=lambda: torch.matmul(aic[:slab], bic), cpu_frac=slab / k,
                 cpu_sample=f"{slab} x {k} x {k} row slab ({slab} of the {k} output rows)"),
        Workload("i32_gemm_256", "1", lambda: mb.matmul(a32, b32, out=o32), (_plain, a32, b32, {}),
                 flops=2.0 * s ** 3, nbytes=4.0 * 3 * s * s, bound="launch",
                 cpu=lambda: torch.matmul(a32c, b32c),
                 note="33.6 M int-ops: launch/latency bound (int32 VALU, no matrix cores)"),
    ]


GROUPS = {
    "headline": group_headline,
    "gemv": group_gemv,
    "layouts": group_layouts,
    "bmm": group_bmm,
    "c64": group_c64,
    "int": group_int,
}

# workload name -> group (for tests and --only)
WORKLOADS = {
    "headline": ["bf16_gemm_8192"],
    "gemv": ["gemv_W@x", "gemv_x@W", "gemv_Wt@x", "gemv_X8@W", "gemv_W@X8"],
    "layouts": [f"bf16_2048x4096x2048_{v}" for v in
                ("rm_rm", "rm_cm", "cm_rm", "cm_cm", "row_sliced", "col_sliced", "offset17", "addmm")],
    "bmm": ["f16_bmm_8x512x512x256", "f16_bmm_broadcastB", "f16_splitk_128x128x65536"],
    "c64": ["c64_gemm_2048_conjA", "c64_gemv_8192"],
    "int": ["i8_gemm_4096", "i32_gemm_256"],
}


# ---------------------------------------------------------------------------------------------
# pricing
# ---------------------------------------------------------------------------------------------

def _sig(x, digits=4):
    """x rounded to `digits` significant digits (keeps the JSON line short)."""
    return float(f"{x:.{digits}g}")


def price(w, ms):
    """The JSON entry of one timed workload (compact: the driver keeps the last 8 KB of the
    line; the parity test of each entry is tests/test_gpu_configs.py::test_config[<name>])."""
    d = {"cfg": w.cfg, "ms": _sig(ms, 5)}
    if w.bound == "hbm":
        gbs = w.nbytes / (ms * 1e-3) / 1e9
        d["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4)}
    elif w.bound == "mfma":
        tf = w.flops / (ms * 1e-3) / 1e12
        unit = "TOP/s" if w.peak_key == "i8" else "TFLOP/s"
        d["roofline"] = {"bound": "mfma", "achieved": round(tf, 2), "peak": PEAK[w.peak_key], "unit": unit,
                         "frac": round(tf / PEAK[w.peak_key], 4)}
    else:
        d["roofline"] = {"bound": "launch", "achieved": round(w.flops / (ms * 1e-3) / 1e9, 1), "unit": "GOP/s"}
    return d


def cpu_threads(args):
    if args.cpu_threads > 0:
        return args.cpu_threads
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return "unknown"


def time_cpu(fn, min_runs=3, min_s=1.0):
    """Best seconds per run: 1 warmup, then at least min_runs runs and at least min_s seconds."""
    fn()
    best, runs, t_all = float("inf"), 0, time.perf_counter()
    while runs < min_runs or time.perf_counter() - t_all < min_s:
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
        runs += 1
    return best, runs


def cpu_entry(w, threads):
    s, runs = time_cpu(w.cpu)
    sec = s / w.cpu_frac     # seconds the whole workload would take at this rate
    if w.bound == "hbm":
        d = {"value": _sig(w.nbytes / sec / 1e9), "unit": "GB/s"}
    elif w.bound == "mfma":
        d = {"value": _sig(w.flops / sec / 1e12), "unit": "TOP/s" if w.peak_key == "i8" else "TFLOP/s"}
    else:
        d = {"value": _sig(w.flops / sec / 1e9), "unit": "GOP/s"}
    if w.cpu_frac != 1.0:
        d["sample"] = w.cpu_sample
    return d, runs


def run_group(torch, mb, name, args, results, want, threads, headline_n):
    builder = GROUPS[name]
    ws = builder(torch, mb, headline_n) if name == "headline" else builder(torch, mb)
    for w in ws:
        if want is not None and w.name not in want:
            continue
        w.call()                      # planning (and the one-shot autotune) outside the timed region
        torch.cuda.synchronize()
        if name == "headline":
            ms = time_events(torch, w.call, args.steps, args.warmup)
        else:
            ms = time_events(torch, w.call, args.steps, args.warmup, CFG_WARM_MS, args.calls)
        entry = price(w, ms)
        if not args.no_cpu and w.cpu is not None:
            entry["cpu_baseline"], runs = cpu_entry(w, threads)
            if name == "headline":
                entry["cpu_runs"] = runs
        results[w.name] = (w, entry)
    del ws
    torch.cuda.empty_cache()


def main(argv=None):
    args = parse(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: run with --gpus 1 (the multi-GPU "
                          "sharding of the path is a design, not a measured configuration)"}))
        sys.exit(2)
    if args.no_tune:
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

    if args.only == "all":
        groups, want = list(GROUPS), None
    elif args.only == "gemm":
        groups, want = ["headline"], None
    elif args.only == "configs":
        groups, want = [g for g in GROUPS if g != "headline"], None
    else:
        items = [s.strip() for s in args.only.split(",") if s.strip()]
        groups = [g for g in GROUPS if g in items or any(n in items for n in WORKLOADS[g])]
        named = {n for g in GROUPS for n in WORKLOADS[g] if n in items}
        want = None if not named else named | {n for g in items if g in WORKLOADS for n in WORKLOADS[g]}
    threads = cpu_threads(args)
    if not args.no_cpu:
        torch.set_num_threads(threads)

    n = args.size
    tuned = os.environ.get("METALBLAS_AUTOTUNE", "1") != "0"
    result = {
        "metric": "TFLOP/s + % MFMA peak (bf16 GEMM 8192³); GEMV HBM GB/s + % peak",
        "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) inputs from torch.Generator seeds, resident in HBM",
        "config": {"workload": f"bf16 GEMM C = A @ B, {n} x {n} x {n}, row-major A and B "
                               "(BASELINE config 3, square case)", "parallelism": "single GPU"},
        "plans": "one-shot autotuner (METALBLAS_AUTOTUNE unset)" if tuned else "static (METALBLAS_AUTOTUNE=0)",
    }
    results = {}
    for gname in groups:
        run_group(torch, mb, gname, args, results, want, threads, n)

    head_name = f"bf16_gemm_{n}"
    if head_name in results:
        w, e = results.pop(head_name)
        ms = e["ms"]
        tf = w.flops / (ms * 1e-3) / 1e12
        result["value"] = round(tf, 2)
        result["ms_per_step"] = round(ms, 4)
        a = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")
        plan = mb.kernels.plan(a, a, out=a, tuned=True)   # the tile the tuner kept, if it ran
        del a
        result["roofline"] = {
            "bound": "mfma", "achieved": round(tf, 2), "peak": PEAK["bf16"], "unit": "TFLOP/s",
            "frac": round(tf / PEAK["bf16"], 4),
            "traffic": TRAFFIC["bf16_gemm_8192"] if n == 8192 else None,
            "kernel": f"matrix-core GEMM tile {plan['tile'][0]}x{plan['tile'][1]} "
                      f"schedule {'ping-pong' if plan['tile'][5] == 2 else 'interleaved'}",
            "algorithmic_per_launch": f"2*{n}^3 = {w.flops:.4e} flop",
            "avg_launch_ms": round(ms, 4),
        }
        result["plan"] = {k: plan[k] for k in ("family", "tile", "split_k", "grid")}
        if "cpu_baseline" in e:
            c = e["cpu_baseline"]
            result["cpu_baseline"] = {"value": c["value"], "unit": c["unit"], "cores": threads,
                                      "kind": "torch.matmul", "model": cpu_model(),
                                      "host_cpus": os.cpu_count(), "runs": e["cpu_runs"],
                                      "sample": f"torch.matmul bf16 on the host CPU, {c['sample']}, "
                                                "1 warmup + best of >= 3 runs and >= 1 s"}
    if results:
        cfg = {}
        for name, (w, e) in results.items():
            e["roofline"]["traffic"] = _sig(TRAFFIC[name]) if name in TRAFFIC else None
            cfg[name] = e
        result["configs"] = cfg
        result["configs_note"] = (
            f"each config: {args.warmup} warmup calls, {CFG_WARM_MS:g} ms of untimed calls, then "
            f"{args.calls or max(args.steps, CFG_MIN_CALLS)} timed calls (HIP events); roofline.traffic = "
            "HBM bytes per launch of the dominant kernel (rocprofv3 FETCH_SIZE/WRITE_SIZE, profiles/); "
            "cpu_baseline = torch.matmul/addmm/bmm on the host CPU "
            f"({threads} threads, best of >= 3 runs and >= 1 s) over the whole workload unless a sample "
            "is named; parity: tests/test_gpu_configs.py::test_config[<name>]")
        if result["value"] is None:
            first = next(iter(cfg.values()))
            result.update({"value": first["roofline"]["achieved"], "unit": first["roofline"]["unit"],
                           "ms_per_step": first["ms"], "roofline": dict(first["roofline"])})
    if not args.no_cpu and "cpu_baseline" not in result and results:
        result["cpu_baseline"] = {"cores": threads, "kind": "torch.matmul", "model": cpu_model(),
                                  "note": "per config, under configs.<name>.cpu_baseline"}
    print(json.dumps(result, separators=(",", ":")))


if __name__ == "__main__":
    main()
