"""One-shot, correctness-guarded autotuner across the kernel families.

Restates the reference's autotuner (metalblas/float_dispatch.py:411-481: ``_probe_params``,
``_fastest``, ``_autotune_mppt``) for gfx950:

  * the C planner's static plan is the primary candidate and runs as planned; its rivals come
    from ``mb_tile_candidates``: the other compiled matrix-core tiles that fit the shape
    (re-derived for 256 CUs and 160 KB of LDS instead of the Apple tables of
    float_dispatch.py:369-404), the thin-product kernels for products with at most 32 rows or
    columns (the reference's gemv_bt / flipt / sgpipe / conv1x1 rivals, float_dispatch.py:
    439-481, 516-542), and coarser / finer K slices of the static tile (its split-K rivals);
  * each candidate runs once and must agree with the primary within 2% of max|C| (exactly,
    for integer dtypes) before it may be timed (float_dispatch.py:464-468);
  * a rival replaces the primary only if it is faster by ``margin`` (3%, as
    float_dispatch.py:157);
  * the winner (None when the static plan stays) is cached per (device, dtype, batch, M, N, K,
    layout, alignment) key; with
    ``METALBLAS_PLAN_CACHE=<file>`` the cache persists as JSON across processes.

As in the reference (float_dispatch.py:156), tuning is on unless ``METALBLAS_AUTOTUNE=0``,
which keeps the C planner's static plans.  The switch is read at each call.  Candidates are
timed into a scratch output with the real output's strides and pointer alignment (so a
column-major or offset ``out`` is tuned as the transposed / offset problem it runs as), with HIP
events on torch's current stream.
"""
from __future__ import annotations

import ctypes
import json
import os
import threading
import time

import torch

from . import _lib

MARGIN = 0.03
_MIN_WORK = 1 << 27          # batch*M*N*K below this is not worth timing
_PLANS: dict = {}
_LOCK = threading.Lock()
_loaded_from: set = set()     # plan-cache files already merged into _PLANS


# os.environ's own bytes dictionary (POSIX): reading it skips the str encode / decode of
# os.environ.get on every call; assignments through os.environ update it
_ENV_DATA = getattr(os.environ, "_data", None)
_ENV_KEY = b"METALBLAS_AUTOTUNE"


def enabled() -> bool:
    if isinstance(_ENV_DATA, dict) and os.name == "posix":
        return _ENV_DATA.get(_ENV_KEY, b"1") != b"0"
    return os.environ.get("METALBLAS_AUTOTUNE", "1") != "0"


def _cache_path():
    return os.environ.get("METALBLAS_PLAN_CACHE") or None


def probe_params(M, N, K):
    """(warmup, iters, reps) scaled down as kernels get longer (float_dispatch.py:411-418)."""
    work = M * N * K
    if work <= 2_000_000_000:
        return 5, 20, 5
    if work <= 50_000_000_000:
        return 3, 10, 5
    return 1, 3, 2


def _load_cache():
    """Merge the plan-cache file named by METALBLAS_PLAN_CACHE into the in-memory plans (once
    per file)."""
    path = _cache_path()
    if not path or path in _loaded_from:
        return
    _loaded_from.add(path)
    if not os.path.exists(path):
        return
    try:
        with open(path) as f:
            data = json.load(f)
        with _LOCK:
            for k, v in data.items():
                _PLANS.setdefault(k, tuple(v) if v is not None else None)
    except (OSError, ValueError):
        pass


def _save_cache():
    path = _cache_path()
    if not path:
        return
    tmp = f"{path}.{os.getpid()}.tmp"
    try:
        with open(tmp, "w") as f:
            json.dump({k: (list(v) if v is not None else None) for k, v in _PLANS.items()}, f)
        os.replace(tmp, path)
    except OSError:
        pass


def _key(desc, device) -> str:
    def layout(m):
        return (int(m.col_stride == 1), int(m.row_stride == 1), int((m.ptr or 0) % 16))
    parts = (device.index if device.index is not None else 0, desc.dtype, desc.batch, desc.M,
             desc.N, desc.K, layout(desc.a), layout(desc.b), layout(desc.c), desc.epilogue)
    return "/".join(map(str, parts))


def clear():
    """Forget every tuned plan (and which plan-cache files were read)."""
    with _LOCK:
        _PLANS.clear()
        _loaded_from.clear()


def cached() -> dict:
    return dict(_PLANS)


# GPU spin (torch.cuda._sleep cycles, which count shader clocks) queued ahead of each timed
# batch: 1.5 x the host time the previous batch took to queue, at up to 3 GHz
_HOLD = [1 << 20]
_HOLD_MIN, _HOLD_MAX = 1 << 18, 1 << 28


def _time_batch(fn, iters):
    """GPU time per call (ms) of ``iters`` back-to-back calls of ``fn``.  A small product's
    call costs more host time (Python, the launch) than GPU time, so events around calls queued
    as the host issues them would time the host.  A spin kernel queued first keeps the GPU busy
    while the calls are queued; if it ended before the last call was queued, the batch is timed
    again (up to four times in all) behind a spin sized from the host time just measured."""
    sleep = getattr(torch.cuda, "_sleep", None)
    for attempt in range(4):
        held = None
        if sleep is not None:
            sleep(_HOLD[0])
            held = torch.cuda.Event()
            held.record()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        host_us = (time.perf_counter() - t0) * 1e6
        late = held is not None and held.query()
        e.record()
        e.synchronize()
        grown = _HOLD[0] >= _HOLD_MAX
        _HOLD[0] = min(_HOLD_MAX, max(_HOLD_MIN, int(host_us * 1.5 * 3000)))
        if not late or grown or attempt == 3:
            return s.elapsed_time(e) / iters


def _fastest(fns, warmup, iters, reps):
    """Per-call times (ms, best of ``reps``) of ``fns``, as the reference's ``_fastest``
    (metalblas/float_dispatch.py:419-433): every candidate's warmup first, then the timed
    repetitions round-robin over the candidates, so a clock that is still ramping up (the
    first call of a shape often comes to an idle GPU) does not favour the candidates timed
    last.  Each repetition times GPU work only (``_time_batch``)."""
    for fn in fns:
        for _ in range(warmup):
            fn()
    torch.cuda.synchronize()
    times = [float("inf")] * len(fns)
    for _ in range(reps):
        for i, fn in enumerate(fns):
            times[i] = min(times[i], _time_batch(fn, iters))
    return times


def apply(desc, choice) -> None:
    """Write a tuned choice (8 ints: a tile request and, in entry 6, a K-slice request; 0 = the
    planner's) into ``desc``."""
    for i in range(6):
        desc.tile[i] = int(choice[i])
    desc.split_k = int(choice[6]) if len(choice) > 6 else 0


def tune(desc, a, b, out, bias=None) -> None:
    """Set ``desc``'s tile (and K-slice) request to the tuned choice for this problem (no-op
    when not applicable or when the static plan won)."""
    if not enabled():
        return
    if desc.batch * desc.M * desc.N * desc.K < _MIN_WORK:
        return
    if torch._C._cuda_isCurrentStreamCapturing():   # timing synchronises: not under graph capture
        return
    _load_cache()
    device = out.device
    key = _key(desc, device)
    with _LOCK:
        hit = key in _PLANS
        choice = _PLANS.get(key)
    if not hit:
        with torch.cuda.device(device):
            choice = _autotune(desc, out)
        with _LOCK:
            _PLANS[key] = choice
            _save_cache()
    if choice is not None:
        apply(desc, choice)


def _like_out(out):
    """A scratch tensor with ``out``'s shape and strides whose data pointer has the same
    alignment modulo 256 bytes, so the candidates run the plan the real output runs (the plan
    depends on the output's layout and on its pointer's low bits)."""
    es = out.element_size()
    span = 1 + sum((n - 1) * abs(st) for n, st in zip(out.shape, out.stride()))
    shift = (out.data_ptr() % 256) // es
    base = torch.empty(span + 256 // es, dtype=out.dtype, device=out.device)
    shift = (shift - (base.data_ptr() % 256) // es) % (256 // es)
    return base.as_strided(out.shape, out.stride(), shift)


def _autotune(desc, out):
    """The fastest of the static plan and its rivals (``mb_tile_candidates``: other matrix-core
    tiles, the thin-product kernels, other K-slice counts), or None when the static plan stays.
    The static plan runs as planned, without a request (a request would turn edge peeling
    off); a rival must agree with it (2% of max|C|, exactly for integers) before it is timed
    and must beat it by MARGIN."""
    cands = _lib.tile_candidates(desc, 24)
    if len(cands) <= 1:
        return None
    lib = _lib.load()
    stream = torch.cuda.current_stream(out.device).cuda_stream
    scratch = _like_out(out)
    ref = _like_out(out)

    def runner(choice, dst):
        d = _lib.MbGemmDesc.from_buffer_copy(desc)
        if choice is not None:
            apply(d, choice)
        if out.dim() == 3:
            d.c = _lib.MbMatrix(ctypes.c_void_p(dst.data_ptr()), dst.stride(1), dst.stride(2), dst.stride(0))
        else:
            d.c = _lib.MbMatrix(ctypes.c_void_p(dst.data_ptr()), dst.stride(0), dst.stride(1), 0)
        nbytes = int(lib.mb_gemm_workspace_bytes(ctypes.byref(d)))
        if nbytes < 0:
            _lib.check(nbytes)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=out.device)
        d.workspace = ctypes.c_void_p(ws.data_ptr())
        d.workspace_bytes = nbytes

        def fn():
            _lib.check(lib.mb_gemm(ctypes.byref(d), ctypes.c_void_p(stream)))
        return fn, ws

    primary_fn, keep0 = runner(None, ref)
    primary_fn()
    torch.cuda.synchronize()
    is_int = out.dtype in (torch.int8, torch.uint8, torch.int16, torch.int32, torch.int64)
    refv = ref.to(torch.complex64 if ref.is_complex() else torch.float32) if not is_int else ref
    scale = float(refv.abs().max().item()) + 1e-6 if not is_int else 0.0

    runs = [(None, primary_fn, keep0)]
    for c in cands[1:]:
        fn, keep = runner(c, scratch)
        fn()
        torch.cuda.synchronize()
        if is_int:
            ok = torch.equal(scratch, ref)
        else:
            sv = scratch.to(refv.dtype)
            ok = bool(torch.isfinite(sv).all().item()) and \
                float((sv - refv).abs().max().item()) <= 0.02 * scale
        if ok:
            runs.append((tuple(c), fn, keep))
    if len(runs) == 1:
        return None
    bt = out.shape[0] if out.dim() == 3 else 1
    warmup, iters, reps = probe_params(bt * desc.M, desc.N, desc.K)
    times = _fastest([fn for _, fn, _ in runs], warmup, iters, reps)
    best = min(range(len(times)), key=times.__getitem__)
    if best and times[best] < times[0] * (1.0 - MARGIN):
        return runs[best][0]
    return None
