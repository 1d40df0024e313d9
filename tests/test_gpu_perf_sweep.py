"""The shape-sweep benchmark (metalblas_amd.perf, the counterpart of the reference's
bench/bench_matmul.py) runs its correctness probe on a shape group and every layout."""
import pytest


@pytest.mark.gpu
def test_sweep_odd_shapes_check(capsys):
    from metalblas_amd import perf
    perf.main(["--group", "odd", "--check"])
    out = capsys.readouterr().out
    assert "FAILED" not in out and "XX" not in out, out
    assert out.count("  ok") == len(perf.SHAPES["odd"])


@pytest.mark.gpu
def test_sweep_layouts_check(capsys):
    from metalblas_amd import perf
    perf.main(["--group", "gemv", "--layout", "all", "--check", "--dtype", "fp16"])
    out = capsys.readouterr().out
    assert "FAILED" not in out and "XX" not in out, out
    assert out.count("  ok") == len(perf.SHAPES["gemv"]) * len(perf.LAYOUTS)


@pytest.mark.gpu
def test_candidates_report(capsys):
    """``--candidates`` times the static plan, every autotune rival and torch on one product."""
    from metalblas_amd import perf
    perf.main(["--candidates", "8x256x256x64"])
    out = capsys.readouterr().out
    assert "static plan" in out and "torch.bmm" in out and out.count("candidate ") >= 2, out


@pytest.mark.gpu
def test_int8_rows_time_int_mm(capsys):
    """int8 rows time torch._int_mm (hipBLASLt, int32 outputs) beside the library's int8 product."""
    from metalblas_amd import perf
    perf.main(["--shape", "512x512x512", "--dtype", "i8", "--check"])
    out = capsys.readouterr().out
    assert "torch._int_mm" in out and "  ok" in out and "FAILED" not in out, out
    assert "median speedup" in out, out
