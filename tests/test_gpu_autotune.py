"""The one-shot autotuner on the GPU (metalblas/float_dispatch.py:411-481 _probe_params /
_fastest / _autotune_mppt, :986-1019 _autotune_bmm), and the persistent plan cache.

Each tuned product is checked against the CPU oracle; the plan cache written by the first
tuning must, after every in-memory plan is forgotten, be read back and reused without timing
anything, giving bit-identical outputs.  Also: the drop-in import name, and ``swizzle_log=``.
"""
import json

import pytest
import torch

import metalblas_amd as mb
from metalblas_amd import dispatch, planner
from helpers import assert_parity, assert_parity_full, gen, rand

pytestmark = pytest.mark.gpu


def _cases(dev):
    """(tag, call, check-args): the benchmark shapes the reference tunes, plus a complex64
    product (its four real products are tuned through the float GEMM in the reference)."""
    g = gen(21)
    a = torch.randn(2048, 4096, generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn(4096, 2048, generator=g).to(torch.bfloat16).to(dev)
    bcm = torch.randn(2048, 4096, generator=g).to(torch.bfloat16).to(dev).t()
    out_cm = torch.empty(2048, 2048, dtype=torch.bfloat16, device=dev).t()   # column-major out
    a3 = torch.randn(8, 512, 256, generator=g).to(torch.float16).to(dev)
    b3 = torch.randn(8, 256, 512, generator=g).to(torch.float16).to(dev)
    ca = rand((1024, 1024), torch.complex64, g).to(dev)
    cb = rand((1024, 1024), torch.complex64, g).to(dev)
    ia = torch.randint(-4, 5, (2048, 2048), generator=g, dtype=torch.int8).to(dev)
    ib = torch.randint(-4, 5, (2048, 2048), generator=g, dtype=torch.int8).to(dev)
    return [
        ("bf16 2048x4096x2048 rm_rm", lambda: mb.matmul(a, b), (a, b)),
        ("bf16 2048x4096x2048 rm_cm", lambda: mb.matmul(a, bcm), (a, bcm)),
        ("bf16 2048x4096x2048 column-major out", lambda: mb.matmul(a, b, out=out_cm), (a, b)),
        ("fp16 bmm 8x512x512x256", lambda: mb.bmm(a3, b3), (a3, b3)),
        ("complex64 1024^3 conj(A)", lambda: mb.matmul(ca.conj(), cb), (ca.conj(), cb)),
        ("int8 2048^3", lambda: mb.matmul(ia, ib), (ia, ib)),
    ]


def test_tuned_plans_match_oracle_and_persist(dev, tmp_path, monkeypatch):
    path = tmp_path / "plans.json"
    monkeypatch.setenv("METALBLAS_AUTOTUNE", "1")
    monkeypatch.setenv("METALBLAS_PLAN_CACHE", str(path))
    planner.clear()
    dispatch.clear_descriptors()
    cases = _cases(dev)
    first = []
    for tag, call, (a, b) in cases:
        print("tuning", tag, flush=True)
        got = call()
        torch.cuda.synchronize()
        assert_parity_full(got, a, b, rows=12, tag=f"tuned {tag}")
        first.append(got.clone())
    tuned = planner.cached()
    assert len(tuned) == len(cases), tuned           # one plan key per case
    assert path.exists()
    on_disk = json.loads(path.read_text())
    assert set(on_disk) == set(tuned)

    # a fresh process's view: no plan in memory, the file named by METALBLAS_PLAN_CACHE
    planner.clear()
    dispatch.clear_descriptors()
    timed = []
    monkeypatch.setattr(planner, "_autotune", lambda *a, **k: timed.append(1))
    for (tag, call, _), want in zip(cases, first):
        got = call()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{tag}: the cached plan gave different bits"
    assert not timed, "a plan in the cache file was tuned again"
    assert planner.cached() == {k: (tuple(v) if v is not None else None) for k, v in on_disk.items()}
    planner.clear()
    dispatch.clear_descriptors()


def test_tuner_off_keeps_static_plans(dev, monkeypatch):
    monkeypatch.setenv("METALBLAS_AUTOTUNE", "0")
    monkeypatch.delenv("METALBLAS_PLAN_CACHE", raising=False)
    planner.clear()
    dispatch.clear_descriptors()
    called = []
    monkeypatch.setattr(planner, "_autotune", lambda *a, **k: called.append(1))
    g = gen(22)
    a = torch.randn(2048, 4096, generator=g).to(torch.bfloat16)
    b = torch.randn(4096, 2048, generator=g).to(torch.bfloat16)
    got = mb.matmul(a.to(dev), b.to(dev))
    assert_parity(got, a, b, tag="static plan")
    assert not called and not planner.cached()
    dispatch.clear_descriptors()


def test_import_name_is_the_references(dev):
    """``import metalblas`` (the reference's package name, pyproject.toml:6) runs this library."""
    import metalblas
    from metalblas.kernels import has_metal4
    assert has_metal4()
    assert metalblas.matmul is mb.matmul and metalblas.bmm is mb.bmm
    g = gen(23)
    a, b = rand((300, 200), torch.bfloat16, g), rand((200, 100), torch.bfloat16, g)
    assert_parity(metalblas.matmul(a.to(dev), b.to(dev)), a, b, tag="import metalblas")


@pytest.mark.parametrize("swz", [0, 1, 2, 3, 5, 6])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=str)
def test_swizzle_log(dev, swz, dtype):
    """``swizzle_log=`` only reorders the tiles (float_dispatch.py:711-717): every value gives
    the same product."""
    g = gen(24 + swz)
    M, N, K = 1100, 1300, 512
    a, b = rand((M, K), dtype, g), rand((K, N), dtype, g)
    got = mb.matmul(a.to(dev), b.to(dev), backend="mpp_tensor", swizzle_log=swz)
    assert_parity(got, a, b, tag=f"swizzle_log={swz} {dtype}")


# products whose static plan is a thin, GEMV or deep-K kernel, or a tile with K slices: the
# tuner's rivals span the kernel families (metalblas/float_dispatch.py:439-481, 516-542)
CROSS = {
    "thin_n 4096x16x4096": (1, 4096, 16, 4096),
    "thin_m 256x4096x4096": (1, 256, 4096, 4096),
    "X8@W 8x16384x4096": (1, 8, 16384, 4096),
    "W@X8 8192x8x8192": (1, 8192, 8, 8192),
    "x@W 1x8192x8192": (1, 1, 8192, 8192),
    "W@x 8192x1x8192": (1, 8192, 1, 8192),
    "deep-K 128x128x32768": (1, 128, 128, 32768),
    "bmm 32x1024x128x1024": (32, 1024, 128, 1024),
}


@pytest.mark.parametrize("case", list(CROSS))
def test_cross_family_candidates_and_tuned_plan_match_oracle(dev, monkeypatch, case):
    """Every rival the tuner may pick (thin-product kernels, the tile family, other K slices),
    forced one by one through the C ABI, matches the oracle; then the tuned call does, and a
    second call of the tuned plan gives the same bits."""
    from metalblas_amd import _lib
    monkeypatch.setenv("METALBLAS_AUTOTUNE", "1")
    monkeypatch.delenv("METALBLAS_PLAN_CACHE", raising=False)
    planner.clear()
    dispatch.clear_descriptors()
    Bb, M, N, K = CROSS[case]
    g = gen(31)
    shape_a, shape_b = ((Bb, M, K), (Bb, K, N)) if Bb > 1 else ((M, K), (K, N))
    a = torch.randn(*shape_a, generator=g).to(torch.bfloat16).to(dev)
    b = torch.randn(*shape_b, generator=g).to(torch.bfloat16).to(dev)
    out = torch.empty(*(shape_a[:-1] + (N,)), dtype=torch.bfloat16, device=dev)
    d = _lib.make_desc(torch.bfloat16, Bb, M, N, K, dispatch._mat(a), dispatch._mat(b), dispatch._mat(out))
    cands = _lib.tile_candidates(d, 24)
    assert len(cands) >= 2, cands
    for c in cands[1:]:
        out.fill_(float("nan"))
        dc = _lib.MbGemmDesc.from_buffer_copy(d)
        planner.apply(dc, c)
        print(f"{case}: candidate {c}", flush=True)
        _lib.run(dc, dev)
        torch.cuda.synchronize()
        assert_parity_full(out, a, b, rows=6, tag=f"{case} candidate {c}")
    got = mb.bmm(a, b) if Bb > 1 else mb.matmul(a, b)
    torch.cuda.synchronize()
    print(f"{case}: tuned choice {list(planner.cached().values())}", flush=True)
    assert_parity_full(got, a, b, rows=6, tag=f"{case} tuned")
    again = mb.bmm(a, b) if Bb > 1 else mb.matmul(a, b)
    assert torch.equal(again, got)
    planner.clear()
    dispatch.clear_descriptors()


def test_tuner_times_gpu_work_not_host_time(dev):
    """A candidate whose calls cost far more host time than GPU time is timed by its GPU work:
    each call here spends 200 us on the host before queuing a ~10 us product."""
    import time
    a = rand((256, 256), torch.bfloat16, gen(3)).to(dev)
    b = rand((256, 256), torch.bfloat16, gen(4)).to(dev)

    def slow_host():
        t = time.perf_counter()
        while time.perf_counter() - t < 2e-4:
            pass
        mb.matmul(a, b)
    for _ in range(3):
        slow_host()
    torch.cuda.synchronize()
    ms = planner._time_batch(slow_host, 10)
    assert ms < 0.1, f"timed {ms * 1e3:.1f} us per call: host time leaked into the GPU timing"
