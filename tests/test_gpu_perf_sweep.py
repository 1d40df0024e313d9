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
