"""The compiled fast path (metalblas_amd/csrc/mb_fast.cpp): a call signature the Python layer has
planned is registered, later calls of it skip Python and must give bit-identical results;
anything else falls through to the Python path."""
import pytest
import torch

import metalblas_amd as mb
from metalblas_amd import dispatch
from helpers import assert_parity, gen, rand

pytestmark = pytest.mark.gpu

needs_fast = pytest.mark.skipif(dispatch._FAST is None, reason="fast path not built")


@needs_fast
@pytest.mark.parametrize("case", ["mm_bf16", "mm_cm", "nd_fold", "bmm_f16", "bmm_broadcast_b", "int8", "int32",
                                  "c64", "split_k", "f32"])
def test_fast_path_matches_python_path(dev, case):
    g = gen(hash(case) % 997)
    if case == "mm_bf16":
        a, b, op = rand((300, 200), torch.bfloat16, g), rand((200, 260), torch.bfloat16, g), "mm"
    elif case == "mm_cm":
        a, b, op = rand((200, 300), torch.float16, g).t(), rand((260, 200), torch.float16, g).t(), "mm"
    elif case == "nd_fold":
        a, b, op = rand((3, 5, 64, 96), torch.bfloat16, g), rand((96, 80), torch.bfloat16, g), "mm"
    elif case == "bmm_f16":
        a, b, op = rand((8, 128, 96), torch.float16, g), rand((8, 96, 112), torch.float16, g), "bmm"
    elif case == "bmm_broadcast_b":
        a, b, op = rand((4, 64, 64), torch.float16, g), rand((64, 48), torch.float16, g).expand(4, 64, 48), "bmm"
    elif case == "int8":
        a, b, op = rand((256, 512), torch.int8, g), rand((512, 128), torch.int8, g), "mm"
    elif case == "int32":
        a, b, op = rand((64, 64), torch.int32, g), rand((64, 64), torch.int32, g), "mm"
    elif case == "c64":
        a, b, op = rand((96, 80), torch.complex64, g), rand((80, 72), torch.complex64, g), "mm"
    elif case == "split_k":
        a, b, op = rand((1, 128, 16384), torch.float16, g), rand((1, 16384, 128), torch.float16, g), "bmm"
    else:
        a, b, op = rand((128, 256), torch.float32, g), rand((256, 64), torch.float32, g), "mm"
    ad = a.to(dev)
    if case == "mm_cm":
        ad = a.t().contiguous().to(dev).t()
        bd = b.t().contiguous().to(dev).t()
    elif case == "bmm_broadcast_b":
        bd = b[0].contiguous().to(dev).expand(4, 64, 48)
    else:
        bd = b.to(dev)
    fn = mb.bmm if op == "bmm" else mb.matmul
    dispatch.clear_descriptors()
    assert dispatch._FAST.size() == 0
    first = fn(ad, bd)                       # Python path: plans, tunes, registers
    assert dispatch._FAST.size() == 1, "the signature was not registered"
    r = dispatch._FAST.bmm(ad, bd) if op == "bmm" else dispatch._FAST.matmul(ad, bd)
    assert r is not None, "a registered signature missed the fast path"
    assert r.shape == first.shape and r.dtype == first.dtype and r.is_contiguous()
    assert torch.equal(r, first), f"{case}: fast path differs from the Python path"
    again = fn(ad, bd)                       # the public call takes the fast path too
    assert torch.equal(again, first)
    if case == "nd_fold":
        assert_parity(again.reshape(-1, 80), a.reshape(-1, 96), b, tag="fast path nd_fold")
    else:
        assert_parity(again, a, b, tag=f"fast path {case}")


@needs_fast
def test_fast_path_falls_through(dev):
    g = gen(5)
    a, b = rand((64, 96), torch.bfloat16, g).to(dev), rand((96, 32), torch.bfloat16, g).to(dev)
    dispatch.clear_descriptors()
    assert dispatch._FAST.matmul(a, b) is None                  # not planned yet
    mb.matmul(a, b)
    assert dispatch._FAST.matmul(a, b) is not None
    assert dispatch._FAST.matmul(a.cpu(), b.cpu()) is None      # CPU tensors
    assert dispatch._FAST.matmul(a, b.to(torch.float16)) is None   # mixed dtypes
    assert dispatch._FAST.matmul(a[:, ::2], b[::2]) is None      # no unit stride: Python copies it
    assert dispatch._FAST.matmul(a[:0], b) is None               # empty
    assert dispatch._FAST.bmm(a, b) is None                      # 2-D into bmm
    c = torch.complex(a.float(), a.float())
    assert dispatch._FAST.matmul(c.conj(), torch.complex(b.float(), b.float())) is None   # conj view
    # another signature (K differs) is not confused with the registered one
    assert dispatch._FAST.matmul(a[:, :64], b[:64]) is None
    # the autotuner switch is part of the signature
    import os
    old = os.environ.get("METALBLAS_AUTOTUNE")
    os.environ["METALBLAS_AUTOTUNE"] = "0"
    try:
        assert dispatch._FAST.matmul(a, b) is None
    finally:
        if old is None:
            del os.environ["METALBLAS_AUTOTUNE"]
        else:
            os.environ["METALBLAS_AUTOTUNE"] = old
    # errors still come from the Python path
    with pytest.raises(AssertionError):
        mb.matmul(a, torch.empty(95, 32, dtype=torch.bfloat16, device=dev))


def test_split_k_workspace_is_per_stream(dev):
    """Split-K products queued on two streams at once, through the compiled path (bmm) and the
    Python path (addmm): each stream has its own scratch, so every result equals its serial one."""
    g = gen(77)
    f16 = torch.float16
    a1, b1 = rand((1, 128, 16384), f16, g).to(dev), rand((1, 16384, 128), f16, g).to(dev)
    a2, b2 = rand((1, 128, 16384), f16, g).to(dev), rand((1, 16384, 128), f16, g).to(dev)
    x1, y1, bias = a1[0], b1[0], rand((128,), f16, g).to(dev)
    assert mb.kernels.plan(a1, b1)["split_k"] > 1
    ref1, ref2 = mb.bmm(a1, b1), mb.bmm(a2, b2)
    ref3 = mb.addmm(bias, x1, y1, beta=0.5, alpha=2.0)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for _ in range(16):
        with torch.cuda.stream(s1):
            outs.append((1, mb.bmm(a1, b1)))
            outs.append((3, mb.addmm(bias, x1, y1, beta=0.5, alpha=2.0)))
        with torch.cuda.stream(s2):
            outs.append((2, mb.bmm(a2, b2)))
            outs.append((3, mb.addmm(bias, x1, y1, beta=0.5, alpha=2.0)))
    torch.cuda.synchronize()
    refs = {1: ref1, 2: ref2, 3: ref3}
    for which, o in outs:
        assert torch.equal(o, refs[which]), f"stream result {which} differs from the serial one"


def test_two_threads_share_one_stream_while_the_workspace_grows(dev):
    """Two host threads queue split-K products of growing size on the same (default) stream
    through the Python path (addmm: an epilogue never takes the compiled fast path).  Each larger
    product replaces the kept split-K workspace while the other thread may sit between picking
    up the old one and queuing its kernels (the C call runs without the GIL); every result must
    still equal, bit for bit, the same call made from one thread."""
    import threading
    from metalblas_amd import _lib
    g = gen(11)
    shapes = [(64, 64, 32768), (128, 128, 32768), (192, 192, 32768), (256, 256, 16384)]
    ops = []
    for m, n, k in shapes:
        a, b = rand((m, k), torch.float16, g).to(dev), rand((k, n), torch.float16, g).to(dev)
        bias = rand((n,), torch.float16, g).to(dev)
        ops.append((bias, a, b))
    want = [mb.addmm(*o, beta=0.5, alpha=2.0) for o in ops]
    torch.cuda.synchronize()
    errors = []

    def worker(order):
        try:
            for rnd in range(6):
                _lib._WS.clear()          # the kept workspace starts small and grows again
                for i in order:
                    got = mb.addmm(*ops[i], beta=0.5, alpha=2.0)
                    if not torch.equal(got, want[i]):
                        errors.append((rnd, shapes[i]))
        except Exception as e:   # pragma: no cover - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(o,)) for o in ([0, 1, 2, 3], [3, 2, 1, 0])]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
