"""Shape-sweep benchmark of ``metalblas_amd.matmul`` against ``torch.matmul`` (hipBLASLt).

The counterpart of the reference's ``bench/bench_matmul.py``: the same shape groups
(``bench/bench_matmul.py:82-101``), operand layouts (``:104-125``), per-layout correctness
probe (``:139-145``) and a per-GPU Markdown report (``:205-259``), timed with HIP events on
this GPU instead of wall clocks around ``torch.mps.synchronize``.

    python -m metalblas_amd.perf                         # bf16, every shape group
    python -m metalblas_amd.perf --group square --dtype fp16
    python -m metalblas_amd.perf --layout all --check    # layout sweep with a parity check
    python -m metalblas_amd.perf --report                # write profiles/shape_sweep_<gpu>.md
    python -m metalblas_amd.perf --bmm --check           # the bmm groups (bench/bench_bmm.py)
    python -m metalblas_amd.perf --trace-summary run_kernel_trace.csv --last 20
    python -m metalblas_amd.perf --candidates 192x512x512x64   # what the autotuner times

The ``torch`` column is ``torch.matmul``; for int8 it is ``torch._int_mm`` (int32 outputs),
torch's only int8 product on the GPU.

Numbers are best-of-``trials`` means over ``iters`` back-to-back calls, so a
power-limited product reports its sustained rate, not its first call.

``--trace-summary`` reads a ``rocprofv3 --kernel-trace --output-format csv`` trace and prints
per-kernel dispatch statistics as a Markdown table; ``--last N`` keeps only each kernel's last N
dispatches (the timed steps of a benchmark whose planning and warmup calls come first).
"""
from __future__ import annotations

import argparse
import os
import statistics
import time

import torch

from . import dispatch as _mb

# the reference's shape groups, (M, N, K) (bench/bench_matmul.py:82-101)
SHAPES = {
    "square": [(s, s, s) for s in (128, 256, 512, 1024, 2048, 4096)],
    "tall": [(4096, 1024, 1024), (1024, 4096, 1024), (8192, 1024, 1024), (2048, 2048, 8192)],
    "attn": [(4096, 4096, 64), (4096, 4096, 128), (4096, 4096, 1024)],
    "gemv": [(1, 4096, 4096), (4096, 1, 4096), (1, 1024, 1024), (1, 32000, 4096)],
    "llm": [(2048, 14336, 4096), (4096, 4096, 11008), (4096, 11008, 4096)],
    "thin_m": [(96, 4096, 4096), (128, 4096, 4096), (192, 4096, 4096), (256, 4096, 4096), (128, 8192, 4096)],
    "thin_n": [(4096, 128, 4096), (4096, 256, 4096), (8192, 128, 4096), (4096, 64, 4096), (4096, 32, 4096),
               (4096, 16, 4096), (4096, 8, 4096)],
    "odd": [(257, 257, 257), (1023, 1023, 1023), (4097, 4097, 4097), (511, 511, 511), (333, 444, 555)],
}

# the reference's bmm shape groups, (B, M, N, K) (bench/bench_bmm.py:51-63)
BMM_SHAPES = {
    "attn": [(96, 512, 512, 64), (96, 512, 64, 512), (192, 512, 512, 64), (192, 512, 64, 512),
             (32, 1024, 1024, 128), (32, 1024, 128, 1024), (48, 2048, 2048, 64)],
    "square": [(64, 128, 128, 128), (64, 256, 256, 256), (32, 512, 512, 512),
               (16, 1024, 1024, 1024), (8, 256, 256, 256), (256, 128, 128, 128)],
    "thin": [(128, 64, 4096, 256), (128, 4096, 64, 256), (256, 32, 2048, 512), (64, 16, 4096, 512)],
    "small": [(512, 64, 64, 64), (1024, 32, 32, 64), (2048, 64, 64, 32)],
}

DTYPES = {
    "fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16, "c64": torch.complex64,
    "c32": torch.complex32, "i8": torch.int8, "u8": torch.uint8, "i16": torch.int16, "i32": torch.int32,
    "i64": torch.int64,
}


def _rand(shape, dtype, gen):
    if dtype.is_complex:
        real = torch.float16 if dtype == torch.complex32 else torch.float32
        re = torch.randn(shape, generator=gen, device="cuda", dtype=real)
        im = torch.randn(shape, generator=gen, device="cuda", dtype=real)
        return torch.complex(re.float(), im.float()).to(dtype)
    if dtype.is_floating_point:
        return torch.randn(shape, generator=gen, device="cuda", dtype=dtype)
    lo = 0 if dtype == torch.uint8 else -4
    return torch.randint(lo, 4, shape, generator=gen, device="cuda", dtype=dtype)


# operand builders for an (r, c) matrix (bench/bench_matmul.py:104-125)
def _rm(r, c, dt, g):
    return _rand((r, c), dt, g)


def _cm(r, c, dt, g):
    return _rand((c, r), dt, g).t()


def _rowsl(r, c, dt, g):
    return _rand((2 * r, c), dt, g)[::2]


def _colsl(r, c, dt, g):
    return _rand((r, 2 * c), dt, g)[:, ::2]


def _off(r, c, dt, g):
    return _rand((r + 1, c + 1), dt, g)[1:, 1:]


LAYOUTS = {
    "rm_rm": (_rm, _rm), "rm_cm": (_rm, _cm), "cm_rm": (_cm, _rm), "cm_cm": (_cm, _cm),
    "sliced": (_rowsl, _rowsl), "colsl": (_colsl, _colsl), "offset": (_off, _off),
}


def _time(fn, iters, trials, warmup):
    """Best-of-trials mean seconds per call (HIP events on the current stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(trials):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        e.synchronize()
        best = min(best, s.elapsed_time(e) * 1e-3 / iters)
    return best


def _plan_iters(flops):
    # about 20 ms of work per trial, at least 5 calls
    return max(5, min(200, int(2e-2 * 1.0e15 / max(flops, 1.0))))


def _ok(a, b, dtype):
    ref = torch.matmul(a.cpu().to(torch.complex128 if dtype.is_complex else
                                  (torch.float64 if dtype.is_floating_point else torch.int64)),
                       b.cpu().to(torch.complex128 if dtype.is_complex else
                                  (torch.float64 if dtype.is_floating_point else torch.int64)))
    got = _mb.matmul(a, b).cpu()
    if not (dtype.is_floating_point or dtype.is_complex):
        # integer products wrap in the accumulator and truncate to the input width
        # (metalblas/integer_dispatch.py:13-19); int64 wraps in the CPU product too
        if dtype == torch.int64:
            return bool(torch.equal(got, ref))
        return bool(torch.equal(got, ref.to(dtype)))
    got = got.to(ref.dtype)
    scale = ref.abs().max().item() or 1.0
    tol = 2e-2 if dtype in (torch.float16, torch.bfloat16, torch.complex32) else 1e-3
    return (got - ref).abs().max().item() <= tol * scale


def bench_one(M, N, K, dtype, build_a=_rm, build_b=_rm, check=False, cool=0.0):
    g = torch.Generator(device="cuda").manual_seed(0)
    a, b = build_a(M, K, dtype, g), build_b(K, N, dtype, g)
    flops = 2.0 * M * N * K * (4.0 if dtype.is_complex else 1.0)
    iters = _plan_iters(flops)
    t0 = time.perf_counter()
    t_torch = None
    if dtype not in (torch.complex32,) and (dtype.is_floating_point or dtype.is_complex):
        t_torch = _time(lambda: torch.matmul(a, b), iters, 5, 3)
    elif dtype == torch.int8 and M > 16 and K % 8 == 0 and N % 8 == 0:
        # torch has no int8 matmul on the GPU; its library product is torch._int_mm (hipBLASLt),
        # which writes int32 outputs (4x the output bytes of the wrapping int8 result)
        t_torch = _time(lambda: torch._int_mm(a, b), iters, 5, 3)
    t_mb = _time(lambda: _mb.matmul(a, b), iters, 5, 3)
    if cool > 0:
        time.sleep(cool * (time.perf_counter() - t0))
    ok = _ok(a, b, dtype) if check else None
    return flops, t_torch, t_mb, ok


def _ok_bmm(a, b, dtype):
    """Sampled batches of a bmm against a CPU float64 product (the bar of _ok)."""
    idx = sorted({0, a.shape[0] // 2, a.shape[0] - 1})
    got = _mb.bmm(a, b)[idx].cpu().double()
    ref = torch.bmm(a[idx].cpu().double(), b[idx].cpu().double())
    tol = 2e-2 if dtype in (torch.float16, torch.bfloat16) else 1e-3
    return (got - ref).abs().max().item() <= tol * (ref.abs().max().item() or 1.0)


def bench_bmm_one(B, M, N, K, dtype, check=False):
    g = torch.Generator(device="cuda").manual_seed(0)
    a = torch.randn(B, M, K, generator=g, device="cuda", dtype=dtype)
    b = torch.randn(B, K, N, generator=g, device="cuda", dtype=dtype)
    flops = 2.0 * B * M * N * K
    iters = _plan_iters(flops)
    t_torch = _time(lambda: torch.bmm(a, b), iters, 5, 3)
    t_mb = _time(lambda: _mb.bmm(a, b), iters, 5, 3)
    ok = _ok_bmm(a, b, dtype) if check else None
    return flops, t_torch, t_mb, ok


def run_bmm_group(name, shapes, dtype, check=False, out=print):
    out(f"\n=== bmm {name}  dtype={str(dtype).replace('torch.', '')} ===")
    out(f"{'B':>4} " + HEADER + ("  chk" if check else ""))
    speedups = []
    for (B, M, N, K) in shapes:
        try:
            flops, tt, tm, ok = bench_bmm_one(B, M, N, K, dtype, check)
            out(_fmt(M, N, K, flops, tt, tm, ok, prefix=f"{B:>4} "))
            speedups.append(tt / tm)
        except Exception as ex:
            out(f"{B:>4} {M:>5} {N:>5} {K:>5} | FAILED: {type(ex).__name__}: {ex}")
    if speedups:
        out(f"median speedup {statistics.median(speedups):.2f}x  (min {min(speedups):.2f}x, max {max(speedups):.2f}x)")
    return speedups


def trace_summary(path, last=0, names=None):
    """Markdown table of a rocprofv3 kernel trace (CSV): calls, average / min / max duration per
    kernel, over each kernel's last ``last`` dispatches when last > 0."""
    import csv
    durs = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = row.get("Kernel_Name") or row.get("KernelName") or row.get("Name")
            t0 = int(row.get("Start_Timestamp") or row.get("BeginNs"))
            t1 = int(row.get("End_Timestamp") or row.get("EndNs"))
            durs.setdefault(name, []).append((t0, t1 - t0))
    lines = ["| kernel | calls | avg us | min us | max us |", "|---|---:|---:|---:|---:|"]
    for name, v in sorted(durs.items(), key=lambda kv: -sum(d for _, d in kv[1])):
        if names and not any(n in name for n in names):
            continue
        v.sort()
        d = [x for _, x in (v[-last:] if last > 0 else v)]
        lines.append(f"| `{name[:150]}` | {len(d)} | {sum(d) / len(d) / 1e3:.2f} | {min(d) / 1e3:.2f} | "
                     f"{max(d) / 1e3:.2f} |")
    return "\n".join(lines)


def pmc_summary(path, kernel, last=0):
    """Per-counter averages of a rocprofv3 --pmc counter_collection CSV over the dispatches of the
    kernels whose name contains ``kernel`` (each kernel's last ``last`` dispatches when last > 0):
    {counter: mean value per dispatch}, plus the number of dispatches averaged under "dispatches"."""
    import csv
    per = {}
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if kernel not in row["Kernel_Name"]:
                continue
            d = per.setdefault(int(row["Dispatch_Id"]), {})
            d[row["Counter_Name"]] = float(row["Counter_Value"])
            if row.get("Start_Timestamp") and row.get("End_Timestamp"):
                d["duration_ns"] = float(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    ids = sorted(per)
    if last > 0:
        ids = ids[-last:]
    out = {}
    for i in ids:
        for c, v in per[i].items():
            out[c] = out.get(c, 0.0) + v / len(ids)
    out["dispatches"] = len(ids)
    return out


# rocprofv3 FETCH_SIZE / WRITE_SIZE scale factors on MI355X: a 1 GiB device copy reads as
# 512 MiB of FETCH_SIZE and 1 GiB of WRITE_SIZE (bench.py --only copy)
FETCH_SCALE, WRITE_SCALE = 2.0, 1.0


def _trace_last(path, kernel, last):
    """Durations (ns) of the last ``last`` dispatches of the kernels whose name contains
    ``kernel`` in a rocprofv3 kernel-trace CSV, and the full name of the first such kernel."""
    import csv
    rows, name = [], None
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            n = row.get("Kernel_Name") or row.get("KernelName") or row.get("Name")
            if kernel not in n:
                continue
            name = name or n
            t0 = int(row.get("Start_Timestamp") or row.get("BeginNs"))
            rows.append((t0, int(row.get("End_Timestamp") or row.get("EndNs")) - t0))
    rows.sort()
    return [d for _, d in (rows[-last:] if last > 0 else rows)], name


def counter_report(trace, pmcs, kernel, last, cus=256, simds=1024, alg_bytes=None, alg_ops=None):
    """Per-dispatch figures of one kernel over its last ``last`` dispatches: duration (kernel
    trace), shader clock (SQ_BUSY_CU_CYCLES / CUs over the duration), matrix-core busy
    (SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x cycles)), LDS instructions and bank-conflict cycles,
    and HBM-side traffic (FETCH_SIZE x 2 + WRITE_SIZE, in bytes) against the algorithmic bytes."""
    durs, name = _trace_last(trace, kernel, last)
    c, ghz = {}, None
    for path in pmcs:
        s = pmc_summary(path, kernel, last)
        if "SQ_BUSY_CU_CYCLES" in s and s.get("duration_ns"):
            ghz = s["SQ_BUSY_CU_CYCLES"] / cus / s["duration_ns"]   # cycles and duration of one run
        for k, v in s.items():
            if k not in ("dispatches", "duration_ns"):
                c[k] = v
    out = {"kernel": name, "dispatches": len(durs)}
    if durs:
        out["us"] = sum(durs) / len(durs) / 1e3
    cyc = c.get("SQ_BUSY_CU_CYCLES", 0.0) / cus
    if ghz:
        out["ghz"] = ghz
    if cyc and "SQ_VALU_MFMA_BUSY_CYCLES" in c:
        out["mfma_busy"] = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * cyc)
    if "SQ_INSTS_LDS" in c:
        out["lds_insts"] = c["SQ_INSTS_LDS"]
        out["lds_conflict_per_inst"] = c.get("SQ_LDS_BANK_CONFLICT", 0.0) / max(c["SQ_INSTS_LDS"], 1.0)
    if "FETCH_SIZE" in c or "WRITE_SIZE" in c:
        out["fetch_bytes"] = c.get("FETCH_SIZE", 0.0) * 1024 * FETCH_SCALE
        out["write_bytes"] = c.get("WRITE_SIZE", 0.0) * 1024 * WRITE_SCALE
        out["traffic"] = out["fetch_bytes"] + out["write_bytes"]
        if alg_bytes:
            out["traffic_x_alg"] = out["traffic"] / alg_bytes
        if durs:
            out["hbm_tbps"] = out["traffic"] / (out["us"] * 1e-6) / 1e12
    if alg_ops and durs:
        out["tops"] = alg_ops / (out["us"] * 1e-6) / 1e12
    out["counters"] = c
    return out


def _fmt(M, N, K, flops, t_torch, t_mb, ok, prefix=""):
    tt = f"{t_torch * 1e3:>9.3f} {flops / t_torch / 1e12:>7.2f}" if t_torch else f"{'-':>9} {'-':>7}"
    sp = f"{t_torch / t_mb:>5.2f}x" if t_torch else f"{'-':>6}"
    chk = "" if ok is None else ("  ok" if ok else "  XX")
    return f"{prefix}{M:>5} {N:>5} {K:>5} | {tt} | {t_mb * 1e3:>9.3f} {flops / t_mb / 1e12:>7.2f} | {sp}{chk}"


HEADER = f"{'M':>5} {'N':>5} {'K':>5} | {'torch ms':>9} {'TFLOPS':>7} | {'mb ms':>9} {'TFLOPS':>7} | speedup"


def run_group(name, shapes, dtype, layout=None, check=False, cool=0.0, out=print):
    build_a, build_b = LAYOUTS[layout or "rm_rm"]
    rows, speedups = [], []
    out(f"\n=== {name}  dtype={str(dtype).replace('torch.', '')}" + (f"  layout={layout}" if layout else "") + " ===")
    if dtype == torch.int8:
        out("(torch column: torch._int_mm, int8 x int8 -> int32; mb: int8 result)")
    out(HEADER + ("  chk" if check else ""))
    for (M, N, K) in shapes:
        try:
            flops, tt, tm, ok = bench_one(M, N, K, dtype, build_a, build_b, check, cool)
            line = _fmt(M, N, K, flops, tt, tm, ok)
            if tt:
                speedups.append(tt / tm)
        except Exception as ex:   # report and go on, like the reference's sweep
            line = f"{M:>5} {N:>5} {K:>5} | FAILED: {type(ex).__name__}: {ex}"
        rows.append(line)
        out(line)
    if speedups:
        out(f"median speedup {statistics.median(speedups):.2f}x  (min {min(speedups):.2f}x, max {max(speedups):.2f}x)")
    return rows, speedups


def candidates(B, M, N, K, dtype=torch.bfloat16, out=print):
    """Time the static plan and every autotune candidate (``mb_tile_candidates``) of one
    row-major product (B > 1: batched), round-robin best-of as the tuner times them, beside
    ``torch.bmm`` / ``torch.matmul``: what the one-shot tuner chooses between for this shape."""
    import ctypes

    from . import _lib, planner
    g = torch.Generator(device="cuda").manual_seed(0)
    a = _rand((B, M, K), dtype, g)
    b = _rand((B, K, N), dtype, g)
    c = torch.empty(B, M, N, dtype=dtype, device="cuda")
    d = _lib.make_desc(dtype, B, M, N, K, (a, K, 1, M * K), (b, N, 1, K * N), (c, N, 1, M * N))
    cands = _lib.tile_candidates(d, 24)
    lib = _lib.load()
    fns = [(lambda: torch.bmm(a, b)) if B > 1 else (lambda: torch.matmul(a[0], b[0]))]
    labels = ["torch.bmm" if B > 1 else "torch.matmul"]
    keep = []
    for i, ch in enumerate(cands):
        dd = _lib.MbGemmDesc.from_buffer_copy(d)
        if i > 0:
            planner.apply(dd, ch)
        info = _lib.plan(dd)
        nb = _lib.workspace_bytes(dd)
        ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
        keep.append(ws)
        dd.workspace = ctypes.c_void_p(ws.data_ptr())
        dd.workspace_bytes = nb
        stream = torch.cuda.current_stream().cuda_stream

        def fn(dd=dd):
            _lib.check(lib.mb_gemm(ctypes.byref(dd), ctypes.c_void_p(stream)))
        fns.append(fn)
        tile = tuple(info.tile[:2])
        sched = {1: "interleaved", 2: "ping-pong", 3: "deep-K"}.get(info.tile[5], f"schedule {info.tile[5] - 1}")
        labels.append(f"{'static plan' if i == 0 else 'candidate'} {tile[0]} x {tile[1]} "
                      f"({info.tile[3]} x {info.tile[4]} waves, {sched}), {info.split_k} K slice(s), "
                      f"grid {tuple(info.grid)}")
    times = planner._fastest(fns, 5, 20, 7)
    flops = 2.0 * B * M * N * K
    out(f"=== candidates  {B} x {M} x {N} x {K}  dtype={str(dtype).replace('torch.', '')} ===")
    for t, lab in sorted(zip(times, labels)):
        out(f"  {t * 1e3:9.2f} us  {flops / t / 1e9:8.1f} TFLOP/s  {lab}")


def machine_info():
    p = torch.cuda.get_device_properties(0)
    return {"gpu": torch.cuda.get_device_name(0), "arch": getattr(p, "gcnArchName", "?"),
            "cus": p.multi_processor_count, "memory_gib": round(p.total_memory / 2 ** 30),
            "torch": torch.__version__, "hip": torch.version.hip}


def write_report(path, dtype=torch.bfloat16, layouts=None, check=False, cool=0.0):
    info = machine_info()
    blocks, all_sp = [], []
    for g, shapes in SHAPES.items():
        lines = []
        rows, sp = run_group(g, shapes, dtype, check=check, cool=cool, out=lines.append)
        blocks.append("\n".join(lines))
        all_sp += sp
    lay_blocks = []
    for lay in layouts or []:
        lines = []
        run_group("square+llm", SHAPES["square"][3:] + SHAPES["llm"], dtype, layout=lay, check=check, cool=cool,
                  out=lines.append)
        lay_blocks.append("\n".join(lines))
    text = [f"# {info['gpu']} ({info['arch']}, {info['cus']} CUs, {info['memory_gib']} GiB)", "",
            f"- torch {info['torch']}, HIP {info['hip']}",
            f"- command: `python -m metalblas_amd.perf --report" + (" --layout " + ",".join(layouts) if layouts else "")
            + (" --check" if check else "") + "`",
            "- times: best of 5 trials of back-to-back calls (about 20 ms each), HIP events; "
            "`torch` is `torch.matmul` (hipBLASLt / rocBLAS)",
            f"- median speedup over all shapes: {statistics.median(all_sp):.2f}x" if all_sp else "", "",
            f"## {str(dtype).replace('torch.', '')} results vs `torch.matmul`", "", "```", "\n\n".join(blocks), "```", ""]
    bmm_blocks, bmm_sp = [], []
    for g, shapes in BMM_SHAPES.items():
        lines = []
        bmm_sp += run_bmm_group(g, shapes, dtype, check=check, out=lines.append)
        bmm_blocks.append("\n".join(lines))
    text += [f"## bmm vs `torch.bmm` (the reference's bench/bench_bmm.py groups)", "",
             f"- median speedup: {statistics.median(bmm_sp):.2f}x" if bmm_sp else "", "", "```",
             "\n\n".join(bmm_blocks), "```", ""]
    if lay_blocks:
        text += ["## Layout sweep (rm = row-major, cm = column-major view, sliced = `[::2]` rows, "
                 "colsl = `[:, ::2]`, offset = `[1:, 1:]`)", "", "```", "\n\n".join(lay_blocks), "```", ""]
    with open(path, "w") as f:
        f.write("\n".join(text))
    return path


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--dtype", default="bf16", choices=list(DTYPES) + ["all"])
    p.add_argument("--group", default="all", choices=list(SHAPES) + list(BMM_SHAPES) + ["all"])
    p.add_argument("--layout", default=None, help="comma list of " + ",".join(LAYOUTS) + " or 'all'")
    p.add_argument("--check", action="store_true", help="compare every result with a CPU fp64/int64 product")
    p.add_argument("--cool", type=float, default=0.0, help="sleep this ratio of each benchmark's time after it")
    p.add_argument("--report", action="store_true", help="write profiles/shape_sweep_<gpu>.md (bf16)")
    p.add_argument("--bmm", action="store_true", help="the bmm shape groups instead of the matmul ones")
    p.add_argument("--shape", metavar="MxNxK", help="one shape instead of the groups (with --layout: each layout)")
    p.add_argument("--candidates", metavar="BxMxNxK", action="append",
                   help="time the static plan and every autotune candidate of this row-major product")
    p.add_argument("--trace-summary", metavar="CSV", help="summarise a rocprofv3 kernel trace and exit")
    p.add_argument("--last", type=int, default=0, help="with --trace-summary: each kernel's last N dispatches")
    p.add_argument("--kernel", action="append", help="with --trace-summary / --pmc-summary: kernels whose name contains this")
    p.add_argument("--pmc-summary", metavar="CSV", nargs="+",
                   help="average rocprofv3 --pmc counter_collection CSVs per dispatch (of --kernel) and exit")
    p.add_argument("--counter-report", metavar="CSV", nargs="+",
                   help="a kernel-trace CSV then --pmc CSVs: one JSON line per --kernel (duration, clock, "
                        "matrix-core busy, LDS conflicts, traffic over the last N dispatches) and exit")
    p.add_argument("--alg-bytes", type=float, default=None, help="with --counter-report: algorithmic bytes")
    p.add_argument("--alg-ops", type=float, default=None, help="with --counter-report: algorithmic flop / op")
    args = p.parse_args(argv)
    if args.counter_report:
        import json
        trace, pmcs = args.counter_report[0], args.counter_report[1:]
        for kern in args.kernel or [""]:
            r = counter_report(trace, pmcs, kern, args.last, alg_bytes=args.alg_bytes, alg_ops=args.alg_ops)
            print(json.dumps(r))
        return
    if args.pmc_summary:
        kern = (args.kernel or [""])[0]
        merged = {}
        for path in args.pmc_summary:
            for c, v in pmc_summary(path, kern, args.last).items():
                if c != "dispatches":
                    merged[c] = v
        print("| counter | mean per dispatch |\n|---|---:|")
        for c in sorted(merged):
            print(f"| `{c}` | {merged[c]:.6g} |")
        return
    if args.trace_summary:
        print(trace_summary(args.trace_summary, args.last, args.kernel))
        return
    if args.candidates:
        for spec in args.candidates:
            shape = tuple(int(v) for v in spec.lower().split("x"))
            if len(shape) != 4:
                p.error("--candidates takes BxMxNxK")
            for dt in (list(DTYPES.values()) if args.dtype == "all" else [DTYPES[args.dtype]]):
                candidates(*shape, dtype=dt)
        return
    layouts = None
    if args.layout:
        layouts = list(LAYOUTS) if args.layout == "all" else args.layout.split(",")
        bad = [x for x in layouts if x not in LAYOUTS]
        if bad:
            p.error(f"unknown layout(s) {bad}; choose from {list(LAYOUTS)} or 'all'")
    if args.report:
        root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
        gpu = machine_info()["arch"].split(":")[0]
        path = os.path.join(root, "profiles", f"shape_sweep_{gpu}.md")
        print("wrote", write_report(path, layouts=layouts, check=args.check, cool=args.cool))
        return
    dtypes = list(DTYPES.values()) if args.dtype == "all" else [DTYPES[args.dtype]]
    if args.bmm:
        groups = list(BMM_SHAPES) if args.group == "all" else [args.group]
        for dt in dtypes:
            for g in groups:
                run_bmm_group(g, BMM_SHAPES[g], dt, check=args.check)
        return
    if args.shape:
        shape = tuple(int(v) for v in args.shape.lower().split("x"))
        if len(shape) != 3:
            p.error("--shape takes MxNxK")
        for dt in dtypes:
            for lay in layouts or [None]:
                run_group("shape", [shape], dt, layout=lay, check=args.check, cool=args.cool)
        return
    groups = list(SHAPES) if args.group == "all" else [args.group]
    for dt in dtypes:
        for g in groups:
            for lay in layouts or [None]:
                run_group(g, SHAPES[g], dt, layout=lay, check=args.check, cool=args.cool)


if __name__ == "__main__":
    main()
