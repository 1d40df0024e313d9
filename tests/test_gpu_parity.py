"""GPU parity: metalblas_amd vs the CPU oracle on the same seeded inputs.

Mirrors the coverage matrix of the reference's tests/test_basic.py:166-255 (forced backends,
transposed layouts, GEMV and strided GEMV, complex64/complex32 with ta/conj, every integer
dtype, addmm bias shapes and scalar combinations, the beta=0 NaN-leak check, bmm /
baddbmm / addbmm, N-D broadcasting, dot/vdot/outer/mv).  Inputs are generated on the CPU
from a seed and copied to the GPU; the oracle sees the same CPU tensors.
"""
import pytest
import torch

import metalblas_amd as mb
from helpers import ALL, COMPLEX, FLOATS, INTS, assert_parity, assert_parity_full, gen, rand

pytestmark = pytest.mark.gpu

BASE = [(64, 64, 64), (128, 128, 128), (256, 256, 256), (513, 257, 129), (1024, 1024, 256)]


def _matrices(M, N, K, dtype, layout, g):
    """tests/test_basic.py:72-82."""
    a = rand((K, M), dtype, g).t() if layout in ("ta", "tr") else rand((M, K), dtype, g)
    b = rand((N, K), dtype, g).t() if layout == "tr" else rand((K, N), dtype, g)
    if layout == "conj":
        a = a.conj()
    elif layout == "strided":
        if N == 1:
            b = rand((K, 2), dtype, g)[:, :1]
        else:
            a = rand((K, 2), dtype, g)[:, :1].t()
    return a, b


def _to(t, dev):
    """Copy to the GPU keeping the view's layout (strides / conj bit)."""
    if t.is_conj():
        return _to(t.conj(), dev).conj()
    base = t.as_strided((t.untyped_storage().nbytes() // t.element_size(),), (1,), 0)
    return base.to(dev).as_strided(t.shape, t.stride(), t.storage_offset())


def check_mm(dev, M, N, K, dtype, backend=None, layout="rm", seed=0):
    g = gen(seed)
    a, b = _matrices(M, N, K, dtype, layout, g)
    kwargs = {"backend": backend} if backend else {}
    got = mb.matmul(_to(a, dev), _to(b, dev), **kwargs)
    assert got.dtype == dtype and got.shape == (M, N)
    assert_parity(got, a, b, tag=f"matmul {dtype} {layout} {backend or 'auto'} {M}x{N}x{K}",
                  strict=backend not in (None, "mpp"))


@pytest.mark.parametrize("dtype", FLOATS, ids=str)
@pytest.mark.parametrize("backend", ["simd", "mpp", "mpp_tensor", "generic", None])
@pytest.mark.parametrize("shape", BASE + [(33, 33, 33)], ids=str)
def test_forced_backends(dev, dtype, backend, shape):
    check_mm(dev, *shape, dtype, backend)


@pytest.mark.parametrize("dtype", FLOATS, ids=str)
@pytest.mark.parametrize("shape", [(128, 128, 128), (513, 257, 129), (1024, 1024, 256),
                                   (1, 4096, 4096), (4096, 1, 4096)], ids=str)
def test_transposed(dev, dtype, shape):
    check_mm(dev, *shape, dtype, layout="tr")


@pytest.mark.parametrize("dtype", FLOATS, ids=str)
@pytest.mark.parametrize("shape", [(1, 4096, 4096), (4096, 1, 4096), (1, 1024, 1024), (1024, 1, 1024)],
                         ids=str)
def test_gemv_backend(dev, dtype, shape):
    check_mm(dev, *shape, dtype, backend="gemv")


@pytest.mark.parametrize("dtype", FLOATS, ids=str)
@pytest.mark.parametrize("shape", [(1, 1024, 256), (1, 4096, 1024), (64, 1, 256), (1024, 1, 1024)], ids=str)
def test_gemv_strided(dev, dtype, shape):
    check_mm(dev, *shape, dtype, backend="gemv", layout="strided")


def test_gemv_backend_rejects_matrix(dev):
    a = torch.randn(8, 8, device=dev)
    with pytest.raises(ValueError):
        mb.matmul(a, a, backend="gemv")
    with pytest.raises(ValueError):
        mb.matmul(a, a, backend="nope")


@pytest.mark.parametrize("shape", [(64, 64, 64), (128, 128, 128), (256, 256, 256), (512, 512, 512),
                                   (1024, 1024, 1024), (513, 257, 129), (333, 444, 555), (2, 64, 128),
                                   (1, 4096, 4096), (4096, 1, 4096), (1, 1024, 1024), (1024, 1, 1024),
                                   (1, 1, 512), (1, 17, 33)], ids=str)
def test_complex64(dev, shape):
    check_mm(dev, *shape, torch.complex64)


@pytest.mark.parametrize("layout", ["ta", "conj"])
@pytest.mark.parametrize("shape", [(256, 256, 256), (513, 257, 129)], ids=str)
def test_complex64_layouts(dev, shape, layout):
    check_mm(dev, *shape, torch.complex64, layout=layout)


@pytest.mark.parametrize("shape", [(256, 256, 256), (512, 512, 512), (1, 2048, 2048), (2048, 1, 2048)], ids=str)
def test_complex32(dev, shape):
    check_mm(dev, *shape, torch.complex32)


@pytest.mark.parametrize("dtype", INTS, ids=str)
@pytest.mark.parametrize("shape", [(64, 64, 64), (256, 256, 256), (513, 257, 129), (333, 444, 555),
                                   (1024, 1024, 1024), (96, 4096, 512), (33, 33, 33), (1, 4096, 4096),
                                   (4096, 1, 4096), (1, 1024, 257), (300, 1, 1024)], ids=str)
def test_integers(dev, dtype, shape):
    check_mm(dev, *shape, dtype)


@pytest.mark.parametrize("dtype", INTS, ids=str)
def test_integers_transposed(dev, dtype):
    check_mm(dev, 256, 256, 256, dtype, layout="ta")


# ---- fused ops (tests/test_basic.py:106-137, 202-242) ----------------------------------------

def check_fused(dev, op, shape, dtype, bshape, beta=1, alpha=1, seed=0):
    g = gen(seed)
    if op == "addmm":
        M, N, K = shape
        a, b = rand((M, K), dtype, g), rand((K, N), dtype, g)
    else:
        Bb, M, N, K = shape
        a, b = rand((Bb, M, K), dtype, g), rand((Bb, K, N), dtype, g)
    bias = rand(bshape, dtype, g)
    got = getattr(mb, op)(bias.to(dev), a.to(dev), b.to(dev), beta=beta, alpha=alpha)
    tag = f"{op} {dtype} {shape} bias={bshape} beta={beta} alpha={alpha}"
    # scalars as metalblas/dispatch.py:127-131 casts them
    if dtype in INTS:
        cb, ca = int(beta), int(alpha)
    elif dtype in COMPLEX:
        cb, ca = beta, alpha
    else:
        cb, ca = float(beta), float(alpha)
    if op == "addbmm":
        Bb, M, N, K = shape
        a2 = a.permute(1, 0, 2).reshape(M, Bb * K)
        b2 = b.reshape(Bb * K, N)
        assert_parity(got, a2, b2, bias=bias, beta=cb, alpha=ca, tag=tag)
    else:
        assert_parity(got, a, b, bias=bias, beta=cb, alpha=ca, tag=tag)


@pytest.mark.parametrize("dtype", ALL, ids=str)
@pytest.mark.parametrize("bshape", [(128, 96), (1, 96), (128, 1), (96,), (1,), ()], ids=str)
def test_addmm_bias_shapes(dev, dtype, bshape):
    check_fused(dev, "addmm", (128, 96, 256), dtype, bshape)


@pytest.mark.parametrize("dtype", ALL, ids=str)
@pytest.mark.parametrize("ba", [(2, 3), (0, 1), (1, 0), (0, 0)], ids=str)
def test_addmm_scalars(dev, dtype, ba):
    check_fused(dev, "addmm", (128, 96, 256), dtype, (96,), *ba)


@pytest.mark.parametrize("dtype", ALL, ids=str)
def test_addmm_gemv(dev, dtype):
    check_fused(dev, "addmm", (1, 4096, 4096), dtype, (4096,))
    check_fused(dev, "addmm", (4096, 1, 4096), dtype, (1,))


@pytest.mark.parametrize("dtype", FLOATS, ids=str)
@pytest.mark.parametrize("mnk", [(130, 100, 200), (257, 257, 257), (333, 444, 555)], ids=str)
def test_addmm_odd(dev, dtype, mnk):
    M, N, K = mnk
    for bshape in [(M, N), (1, N), (M, 1), (N,), (1,), ()]:
        check_fused(dev, "addmm", (M, N, K), dtype, bshape)


@pytest.mark.parametrize("dtype", FLOATS, ids=str)
def test_addmm_beta0_nan_bias(dev, dtype):
    """tests/test_basic.py:214-217: beta == 0 must not read the bias."""
    g = gen(0)
    a, b = rand((128, 256), dtype, g).to(dev), rand((256, 96), dtype, g).to(dev)
    got = mb.addmm(torch.full((128, 96), float("nan"), dtype=dtype, device=dev), a, b, beta=0)
    assert not torch.isnan(got).any().item()


BMM_SHAPES = [(8, 128, 128, 128), (32, 256, 256, 256), (4, 512, 512, 512), (96, 512, 512, 64),
              (16, 64, 4096, 512), (128, 4096, 64, 256), (512, 64, 64, 64), (2048, 64, 64, 32),
              (3, 130, 100, 200), (8, 1, 512, 256), (8, 512, 1, 256)]


def check_bmm(dev, Bb, M, N, K, dtype, layout="rm", seed=0):
    g = gen(seed)
    if layout == "tr":
        a = rand((Bb, K, M), dtype, g).transpose(-2, -1)
        b = rand((Bb, N, K), dtype, g).transpose(-2, -1)
    else:
        a, b = rand((Bb, M, K), dtype, g), rand((Bb, K, N), dtype, g)
    got = mb.bmm(_to(a, dev), _to(b, dev))
    assert_parity(got, a, b, tag=f"bmm {dtype} {layout} {Bb}x{M}x{N}x{K}")


@pytest.mark.parametrize("dtype", ALL, ids=str)
@pytest.mark.parametrize("shape", BMM_SHAPES, ids=str)
def test_bmm(dev, dtype, shape):
    check_bmm(dev, *shape, dtype)


@pytest.mark.parametrize("dtype", ALL, ids=str)
def test_bmm_transposed(dev, dtype):
    check_bmm(dev, 8, 256, 256, 256, dtype, "tr")


@pytest.mark.parametrize("case", [(torch.bfloat16, 36, 2048, 2048, 64), (torch.float16, 24, 2000, 3008, 96),
                                  (torch.int8, 17, 4096, 4096, 128)], ids=str)
def test_bmm_streamed_output(dev, case):
    """Outputs past the 256 MiB last-level cache (302, 289 and 285 MB) leave the LDS-staged
    epilogue through non-temporal stores: whole 256 x 256 tiles with one K stage, a ragged last
    tile row with a K edge (fp16), and 8-bit outputs (16 per chunk, bit-exact)."""
    dtype, Bb, M, N, K = case
    g = gen(77)
    a, b = rand((Bb, M, K), dtype, g).to(dev), rand((Bb, K, N), dtype, g).to(dev)
    assert Bb * M * N * a.element_size() >= 256 << 20
    got = mb.bmm(a, b)
    assert_parity_full(got, a, b, rows=16, tag=f"bmm streamed {case}")


@pytest.mark.parametrize("dtype", ALL, ids=str)
@pytest.mark.parametrize("bshape", [(4, 128, 96), (4, 1, 96), (4, 128, 1), (1, 128, 96), (128, 96), (96,),
                                    (1,), ()], ids=str)
def test_baddbmm_bias_shapes(dev, dtype, bshape):
    check_fused(dev, "baddbmm", (4, 128, 96, 256), dtype, bshape)


@pytest.mark.parametrize("dtype", ALL, ids=str)
@pytest.mark.parametrize("ba", [(2, 3), (0, 1), (1, 0), (0, 0)], ids=str)
def test_baddbmm_scalars(dev, dtype, ba):
    check_fused(dev, "baddbmm", (4, 128, 96, 256), dtype, (96,), *ba)


@pytest.mark.parametrize("dtype", ALL, ids=str)
def test_addbmm(dev, dtype):
    for bshape in [(128, 96), (1, 96), (128, 1), (96,), (1,), ()]:
        check_fused(dev, "addbmm", (8, 128, 96, 256), dtype, bshape)
    for shape in [(32, 64, 64, 64), (4, 256, 256, 512)]:
        check_fused(dev, "addbmm", shape, dtype, (shape[2],))
    for ba in [(1, 1), (2, 3), (0, 1), (1, 0)]:
        check_fused(dev, "addbmm", (8, 128, 96, 256), dtype, (96,), *ba)


@pytest.mark.parametrize("dtype", FLOATS, ids=str)
@pytest.mark.parametrize("mnk", [(130, 100, 200), (257, 129, 257)], ids=str)
def test_baddbmm_odd(dev, dtype, mnk):
    M, N, K = mnk
    for bshape in [(4, M, N), (N,), ()]:
        check_fused(dev, "baddbmm", (4, M, N, K), dtype, bshape)


# ---- N-D broadcasting and vector helpers (tests/test_basic.py:140-163, 244-255) ------------

ND_CASES = [((64,), (64,)), ((32,), (32, 48)), ((40, 32), (32,)), ((32,), (8, 32, 48)),
            ((6, 40, 32), (32,)), ((8, 40, 32), (8, 32, 48)), ((8, 40, 32), (32, 48)),
            ((40, 32), (8, 32, 48)), ((2, 3, 40, 32), (2, 3, 32, 48)), ((3, 1, 64, 32), (1, 5, 32, 48)),
            ((2, 3, 40, 32), (32, 48))]


def _torch_ref_nd(a, b):
    """Broadcast with torch on CPU, then run the oracle on the 3-D/2-D form."""
    a2 = a.unsqueeze(0) if a.dim() == 1 else a
    b2 = b.unsqueeze(-1) if b.dim() == 1 else b
    batch = torch.broadcast_shapes(a2.shape[:-2], b2.shape[:-2])
    M, K = a2.shape[-2:]
    N = b2.shape[-1]
    return a2, b2, batch, M, N, K


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.int32], ids=str)
@pytest.mark.parametrize("view", ["contiguous", "row_sliced", "batch_transposed"])
def test_nd_fold_into_rows(dev, dtype, view):
    """(..., M, K) @ (K, N): A's leading dims fold into its rows when that is a view (one 2-D
    product), else the broadcast-batch path; both give the batched result."""
    g = gen(5)
    if view == "contiguous":
        a = rand((4, 96, 64), dtype, g)
    elif view == "row_sliced":
        a = rand((4, 192, 64), dtype, g)[:, ::2]
    else:
        a = rand((96, 4, 64), dtype, g).transpose(0, 1)
    b = rand((64, 80), dtype, g)
    got = mb.matmul(_to(a, dev), b.to(dev))
    assert got.shape == (4, 96, 80) and got.dtype == dtype
    assert_parity(got, a, b.expand(4, 64, 80), tag=f"nd fold {dtype} {view}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.complex64,
                                   torch.int32, torch.int8, torch.int64], ids=str)
@pytest.mark.parametrize("shapes", ND_CASES, ids=str)
def test_nd_broadcast(dev, dtype, shapes):
    g = gen(0)
    a, b = rand(shapes[0], dtype, g), rand(shapes[1], dtype, g)
    got = mb.matmul(a.to(dev), b.to(dev))
    expect_shape = torch.matmul(a.to(torch.float32 if dtype not in COMPLEX else torch.complex64),
                                b.to(torch.float32 if dtype not in COMPLEX else torch.complex64)).shape
    assert got.shape == expect_shape and got.dtype == dtype
    a2, b2, batch, M, N, K = _torch_ref_nd(a, b)
    if batch:
        size = 1
        for s in batch:
            size *= s
        a3 = a2.expand(*batch, M, K).reshape(size, M, K)
        b3 = b2.expand(*batch, K, N).reshape(size, K, N)
        assert_parity(got.reshape(size, M, N), a3, b3, tag=f"nd {dtype} {shapes}")
    else:
        assert_parity(got.reshape(M, N), a2, b2, tag=f"nd {dtype} {shapes}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.complex64,
                                   torch.complex32, torch.int8, torch.int32, torch.int64], ids=str)
def test_vectors(dev, dtype):
    g = gen(0)
    for k in (4096, 7, 1):
        a, b = rand((k,), dtype, g), rand((k,), dtype, g)
        got = mb.dot(a.to(dev), b.to(dev))
        assert got.shape == () and got.dtype == dtype
        assert_parity(got.reshape(1, 1), a.reshape(1, k), b.reshape(k, 1), tag=f"dot {dtype} {k}")
        got = mb.vdot(a.to(dev), b.to(dev))
        assert got.shape == ()
        assert_parity(got.reshape(1, 1), a.reshape(1, k).conj() if dtype in COMPLEX else a.reshape(1, k),
                      b.reshape(k, 1), tag=f"vdot {dtype} {k}")
    a, b = rand((128,), dtype, g), rand((96,), dtype, g)
    got = mb.outer(a.to(dev), b.to(dev))
    assert got.shape == (128, 96)
    assert_parity(got, a.reshape(128, 1), b.reshape(1, 96), k=1, tag=f"outer {dtype}")
    a, b = rand((256, 512), dtype, g), rand((512,), dtype, g)
    got = mb.mv(a.to(dev), b.to(dev))
    assert got.shape == (256,)
    assert_parity(got.reshape(256, 1), a, b.reshape(512, 1), tag=f"mv {dtype}")


def test_empty_and_k0(dev):
    """metalblas/dispatch.py:215-218: empty batch -> empty, K == 0 -> zeros."""
    a = torch.randn(3, 4, 0, device=dev)
    b = torch.randn(3, 0, 5, device=dev)
    r = mb.bmm(a, b)
    assert r.shape == (3, 4, 5) and bool((r == 0).all())
    r = mb.bmm(torch.randn(0, 4, 2, device=dev), torch.randn(0, 2, 5, device=dev))
    assert r.shape == (0, 4, 5)
    bias = torch.randn(5, device=dev)
    r = mb.addmm(bias, torch.randn(4, 0, device=dev), torch.randn(0, 5, device=dev), beta=2.0)
    assert torch.allclose(r, (2.0 * bias).expand(4, 5))


# ---- thin products: every GEMV family, both operand layouts, 1..16 vectors --------------------

THIN_NV = [1, 2, 3, 5, 8, 12, 16]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.int8,
                                   torch.int32, torch.complex64], ids=str)
@pytest.mark.parametrize("nv", THIN_NV)
@pytest.mark.parametrize("layout", ["rr", "rc", "cr", "cc"])
def test_thin_n(dev, dtype, nv, layout):
    """W @ X with a thin X (N = nv): W row/col-major, X row/col-major."""
    g = gen(nv)
    M, K = 1024, 2048
    a = rand((M, K), dtype, g) if layout[0] == "r" else rand((K, M), dtype, g).t()
    b = rand((K, nv), dtype, g) if layout[1] == "r" else rand((nv, K), dtype, g).t()
    got = mb.matmul(_to(a, dev), _to(b, dev))
    assert_parity(got, a, b, tag=f"thin-N {dtype} nv={nv} {layout}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.int8,
                                   torch.int32, torch.complex64], ids=str)
@pytest.mark.parametrize("nv", THIN_NV)
@pytest.mark.parametrize("layout", ["rr", "rc", "cr", "cc"])
def test_thin_m(dev, dtype, nv, layout):
    """X @ W with a thin X (M = nv)."""
    g = gen(100 + nv)
    N, K = 1024, 2048
    a = rand((nv, K), dtype, g) if layout[0] == "r" else rand((K, nv), dtype, g).t()
    b = rand((K, N), dtype, g) if layout[1] == "r" else rand((N, K), dtype, g).t()
    got = mb.matmul(_to(a, dev), _to(b, dev))
    assert_parity(got, a, b, tag=f"thin-M {dtype} nv={nv} {layout}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
@pytest.mark.parametrize("shape", [(4096, 8, 4096), (8, 4096, 4096), (3000, 1, 2048), (1, 3000, 2048)], ids=str)
def test_thin_addmm(dev, dtype, shape):
    M, N, K = shape
    g = gen(7)
    a, b = rand((M, K), dtype, g), rand((K, N), dtype, g)
    bias = rand((N,), dtype, g)
    got = mb.addmm(bias.to(dev), a.to(dev), b.to(dev), beta=0.5, alpha=2.0)
    assert_parity(got, a, b, bias=bias, beta=0.5, alpha=2.0, tag=f"thin addmm {dtype} {shape}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("nv", [2, 3, 5, 8, 12, 16])
@pytest.mark.parametrize("layout", ["rr", "rc", "cr", "cc"])
@pytest.mark.parametrize("side", ["N", "M"])
def test_thin_matrix_cores(dev, dtype, nv, layout, side):
    """Thin products with a large matrix run on the matrix cores: k_thin_dot4 (4 x 16,
    K-contiguous matrix, from 5 vectors) or k_thin16 (32 x 256, N-contiguous matrix), split-K,
    vectors copied K-contiguous when they are not: wide side 2304 (a partial tile), K = 2088
    (a partial stage / K quarter)."""
    g = gen(300 + nv)
    wide, K = 2304, 2088
    if side == "N":
        a = rand((wide, K), dtype, g) if layout[0] == "r" else rand((K, wide), dtype, g).t()
        b = rand((K, nv), dtype, g) if layout[1] == "r" else rand((nv, K), dtype, g).t()
    else:
        a = rand((nv, K), dtype, g) if layout[0] == "r" else rand((K, nv), dtype, g).t()
        b = rand((K, wide), dtype, g) if layout[1] == "r" else rand((wide, K), dtype, g).t()
    ad, bd = _to(a, dev), _to(b, dev)
    p = mb.kernels.plan(ad, bd)
    dot = (side == "N" and layout[0] == "r") or (side == "M" and layout[1] == "c")   # K-contiguous matrix
    if (nv >= 5 or nv == 3) if dot else nv >= 2:
        assert p["family"] == "mfma" and (p["tile"][:2] == (4, 16) if dot else p["tile"][0] == 32), p
    got = mb.matmul(ad, bd)
    assert_parity(got, a, b, tag=f"thin mfma {dtype} nv={nv} {layout} {side}")


@pytest.mark.parametrize("case", ["bmm", "broadcast", "addmm", "kodd"])
def test_thin_matrix_cores_more(dev, case):
    """Batched and broadcast thin products, the fused epilogue, and an odd K (the matrix
    cannot be streamed in place: the GEMV path takes it)."""
    g = gen(11)
    dt = torch.bfloat16
    if case == "bmm":
        a, b = rand((3, 2304, 2088), dt, g), rand((3, 2088, 8), dt, g)
        assert_parity(mb.bmm(a.to(dev), b.to(dev)), a, b, tag="thin bmm")
    elif case == "broadcast":
        a, b = rand((3, 4, 2088), dt, g), rand((2088, 2304), dt, g)
        got = mb.matmul(a.to(dev), b.to(dev))
        assert_parity(got, a, b.expand(3, 2088, 2304), tag="thin broadcast")
    elif case == "addmm":
        a, b, bias = rand((2304, 2088), dt, g), rand((2088, 6), dt, g), rand((6,), dt, g)
        got = mb.addmm(bias.to(dev), a.to(dev), b.to(dev), beta=0.5, alpha=-1.5)
        assert_parity(got, a, b, bias=bias, beta=0.5, alpha=-1.5, tag="thin addmm mfma")
    else:
        a, b = rand((2304, 2051), dt, g), rand((2051, 8), dt, g)
        assert mb.kernels.plan(a.to(dev), b.to(dev))["family"] != "mfma"
        assert_parity(mb.matmul(a.to(dev), b.to(dev)), a, b, tag="thin odd K")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", [(16, 16, 2048, 512, None), (64, 24, 1024, 256, None), (256, 16, 1024, 64, None),
                                  (128, 16, 1024, 1024, None), (1, 16, 16384, 1024, None),
                                  (1, 1, 16384, 2048, None), (1, 1, 4096, 4096, None),
                                  (1, 32, 2304, 520, (32, 256)), (1, 16, 1024, 40, (32, 256)),
                                  (1, 5, 1000, 136, (32, 256)), (1, 32, 2304, 520, (32, 128)),
                                  (1, 16, 1024, 40, (32, 128)), (1, 5, 1000, 136, (32, 128))], ids=str)
@pytest.mark.parametrize("a_layout", ["r", "c"])
def test_thin_rows_batched_and_short_k(dev, dtype, case, a_layout):
    """The 32 x 256 and 32 x 128 matrix-core tiles for up to 32 vectors (rows of A) over an
    N-contiguous matrix: batched and short-K products (no K slices, a single stage), a ragged K
    (partial stage), a ragged N edge, and A copied K-contiguous when it is column-major.
    Explicit tile requests (2-D) skip the size rules; the automatic cases are ones the planner
    routes to these tiles."""
    B, M, N, K, tile = case
    g = gen(M * 7 + K)
    if a_layout == "r":
        a = rand((B, M, K), dtype, g)
    else:
        a = rand((B, K, M), dtype, g).transpose(1, 2)
    b = rand((B, K, N), dtype, g)
    if B == 1:
        a, b = a[0], b[0]
    ad, bd = _to(a, dev), _to(b, dev)
    p = mb.kernels.plan(ad, bd, tile=tile)
    assert p["family"] == "mfma" and p["tile"][0] == 32 and p["tile"][1] == (tile[1] if tile else p["tile"][1]), p
    assert p["tile"][1] in (128, 256), p
    if B > 1:
        got = mb.bmm(ad, bd)
    else:
        got = mb.matmul(ad, bd, tile=tile) if tile else mb.matmul(ad, bd)
    assert_parity(got, a, b, tag=f"thin rows {dtype} {case} A {a_layout}")


@pytest.mark.parametrize("n", [8192, 16384])
def test_gemv_config2_sizes(dev, n):
    """Benchmark config 2 at full size: y = W @ x, x @ W and 8-vector thin products,
    checked on sampled rows against the oracle."""
    g = gen(1)
    W = torch.randn(n, n, generator=g).to(torch.bfloat16)
    x = torch.randn(n, generator=g).to(torch.bfloat16)
    Wd, xd = W.to(dev), x.to(dev)
    assert_parity(mb.matmul(Wd, xd).reshape(n, 1), W, x.reshape(n, 1), tag="W@x")
    assert_parity(mb.matmul(xd, Wd).reshape(1, n), x.reshape(1, n), W, tag="x@W")
    X8 = torch.randn(8, n, generator=g).to(torch.bfloat16)
    assert_parity(mb.matmul(X8.to(dev), Wd), X8, W, tag="X8@W")
    Xn = torch.randn(n, 8, generator=g).to(torch.bfloat16)
    assert_parity(mb.matmul(Wd, Xn.to(dev)), W, Xn, tag="W@X8")


# ---- every compiled 16-bit matrix-core schedule, forced, on edge shapes and all layouts ---------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.int8, torch.uint8], ids=str)
@pytest.mark.parametrize("tile", [(256, 256, 64, 2, 4, 1), (256, 256, 64, 2, 4, 2), (256, 128, 64, 2, 4, 2),
                                  (256, 256, 64, 2, 2, 1), (128, 128, 64, 2, 2, 1), (64, 64, 64, 2, 2, 1),
                                  (64, 64, 64, 2, 2, 3)], ids=str)
@pytest.mark.parametrize("shape", [(256, 256, 64), (513, 257, 129), (1000, 700, 1000), (512, 768, 4160),
                                   (64, 64, 4096)], ids=str)
@pytest.mark.parametrize("layout", ["rr", "rc", "cr", "cc"])
def test_matrix_core_schedules(dev, dtype, tile, shape, layout):
    M, N, K = shape
    g = gen(hash((M, N, K, layout)) % 1000)
    a = rand((M, K), dtype, g) if layout[0] == "r" else rand((K, M), dtype, g).t()
    b = rand((K, N), dtype, g) if layout[1] == "r" else rand((N, K), dtype, g).t()
    got = mb.matmul(_to(a, dev), _to(b, dev), backend="mpp", tile=tile)
    assert_parity(got, a, b, tag=f"tile {tile} {dtype} {layout} {shape}")


# ---- operands the matrix-core loaders cannot stream in place (copied into the workspace) ------

def _offset_view(shape, dtype, g, offset, transpose=False, ld_pad=0):
    """A matrix view at a storage offset and/or with a padded leading dimension."""
    rows, cols = (shape[1], shape[0]) if transpose else shape
    ld = cols + ld_pad
    base = rand((offset + rows * ld,), dtype, g)
    v = base[offset:].as_strided((rows, cols), (ld, 1))
    return v.t() if transpose else v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.int8, torch.uint8], ids=str)
@pytest.mark.parametrize("case", ["offset17_a", "offset1_b", "odd_ld_a", "odd_k", "both_cm_offset",
                                  "batched_offset", "ref_offset_k516", "ref_offset_k517"])
def test_unaligned_operands(dev, dtype, case):
    g = gen(17)
    M, N, K = 384, 320, 512
    if case == "offset17_a":
        a, b = _offset_view((M, K), dtype, g, 17), rand((K, N), dtype, g)
    elif case == "offset1_b":
        a, b = rand((M, K), dtype, g), _offset_view((K, N), dtype, g, 1)
    elif case == "odd_ld_a":
        a, b = _offset_view((M, K), dtype, g, 0, ld_pad=3), rand((K, N), dtype, g)
    elif case == "odd_k":
        K = 517
        a, b = rand((M, K), dtype, g), rand((K, N), dtype, g)
    elif case == "both_cm_offset":
        a = _offset_view((M, K), dtype, g, 5, transpose=True)
        b = _offset_view((K, N), dtype, g, 3, transpose=True)
    elif case.startswith("ref_offset"):
        # the reference benchmark's 'offset' layout, [1:, 1:] of (rows + 1) x (cols + 1)
        # (bench/bench_matmul.py:120-121): K = 516 gives rows alternating between word-aligned
        # and half-word starts, K = 517 rows that end inside a 16-byte chunk
        K = int(case[-3:])
        a = rand((M + 1, K + 1), dtype, g)[1:, 1:]
        b = rand((K + 1, N + 1), dtype, g)[1:, 1:]
    else:
        Bb = 3
        base = rand((9 + Bb * M * K,), dtype, g)
        a = base[9:].view(Bb, M, K)
        b = rand((Bb, K, N), dtype, g)
        got = mb.bmm(_to(a, dev), _to(b, dev))
        assert_parity(got, a, b, tag=f"unaligned {case} {dtype}")
        return
    got = mb.matmul(_to(a, dev), _to(b, dev))
    plan = mb.kernels.plan(_to(a, dev), _to(b, dev))
    assert plan["family"] == "mfma", plan
    assert_parity(got, a, b, tag=f"unaligned {case} {dtype} {tuple(a.stride())} off {a.storage_offset()}")


def test_unaligned_addmm_config3_offset(dev):
    """Benchmark config 3 'offset' layout: a contiguous view at storage offset 17, with addmm."""
    g = gen(3)
    M, K, N = 1024, 2048, 768
    flat = rand((17 + M * K,), torch.bfloat16, g)
    a = flat[17:].view(M, K)
    b = rand((K, N), torch.bfloat16, g)
    bias = rand((N,), torch.bfloat16, g)
    got = mb.addmm(bias.to(dev), _to(a, dev), b.to(dev), beta=0.5, alpha=2.0)
    assert_parity(got, a, b, bias=bias, beta=0.5, alpha=2.0, tag="offset17 addmm")


@pytest.mark.parametrize("dtype", [torch.int8, torch.uint8], ids=str)
@pytest.mark.parametrize("layout", ["rr", "rc", "cr", "cc"])
@pytest.mark.parametrize("tile", [None, (256, 256, 64, 2, 4, 2), (128, 128, 64, 2, 2, 1)], ids=str)
def test_int8_full_range(dev, dtype, layout, tile):
    """Full-range 8-bit operands through the int8 matrix cores: signed and unsigned values,
    products wrapping modulo 2^8 on the store, and the fused integer epilogue."""
    g = gen(88)
    M, N, K = 512, 384, 1152
    lo, hi = (-128, 128) if dtype is torch.int8 else (0, 256)
    def full(shape):
        return torch.randint(lo, hi, shape, generator=g, dtype=torch.int64).to(dtype)
    a = full((M, K)) if layout[0] == "r" else full((K, M)).t()
    b = full((K, N)) if layout[1] == "r" else full((N, K)).t()
    kw = {} if tile is None else {"backend": "mpp", "tile": tile}
    got = mb.matmul(_to(a, dev), _to(b, dev), **kw)
    assert_parity(got, a, b, tag=f"int8 full {dtype} {layout} {tile}")
    bias = full((N,))
    got = mb.addmm(bias.to(dev), _to(a, dev), _to(b, dev), beta=3, alpha=-5)
    assert_parity(got, a, b, bias=bias, beta=3, alpha=-5, tag=f"int8 addmm {dtype} {layout}")


# ---- complex products on the real matrix cores (expanded B, interleaved A) --------------------

@pytest.mark.parametrize("dtype", [torch.complex64, torch.complex32], ids=str)
@pytest.mark.parametrize("conj", ["none", "a", "b", "ab"])
@pytest.mark.parametrize("layout", ["rr", "cr", "rc", "cc"])
def test_complex_matrix_cores(dev, dtype, conj, layout):
    g = gen(33)
    M, N, K = 320, 288, 260
    a = rand((M, K), dtype, g) if layout[0] == "r" else rand((K, M), dtype, g).t()
    b = rand((K, N), dtype, g) if layout[1] == "r" else rand((N, K), dtype, g).t()
    if "a" in conj:
        a = a.conj()
    if "b" in conj:
        b = b.conj()
    got = mb.matmul(_to(a, dev), _to(b, dev))
    assert mb.kernels.plan(_to(a, dev).resolve_conj(), _to(b, dev).resolve_conj())["family"] == "mfma"
    assert_parity(got, a, b, tag=f"complex mfma {dtype} conj={conj} {layout}")


@pytest.mark.parametrize("dtype", [torch.complex64, torch.complex32], ids=str)
def test_complex_matrix_cores_fused(dev, dtype):
    """Complex epilogue through the complex reduction, column-major output, odd K, batches."""
    g = gen(34)
    M, N, K = 256, 320, 257
    a, b = rand((M, K), dtype, g), rand((K, N), dtype, g)
    bias = rand((N,), dtype, g)
    beta, alpha = complex(0.5, -1.0), complex(2.0, 0.25)
    got = mb.addmm(bias.to(dev), a.to(dev), b.to(dev), beta=beta, alpha=alpha)
    assert_parity(got, a, b, bias=bias, beta=beta, alpha=alpha, tag=f"complex addmm {dtype}")
    out = torch.empty(N, M, dtype=dtype, device=dev).t()
    mb.matmul(a.to(dev), b.to(dev), out=out)
    assert_parity(out, a, b, tag=f"complex cm out {dtype}")
    a3, b3 = rand((3, M, K), dtype, g), rand((3, K, N), dtype, g)
    assert_parity(mb.bmm(a3.to(dev), b3.to(dev)), a3, b3, tag=f"complex bmm {dtype}")
    bb = rand((K, N), dtype, g)
    got = mb.matmul(a3.to(dev), bb.to(dev))
    assert_parity(got, a3, bb.expand(3, K, N), tag=f"complex broadcast {dtype}")


# ---- products peeled into whole 256 x 256 tiles plus 1..16-row (column) strips --------------

@pytest.mark.parametrize("case", [("bf16", 4097, 4096, 4096, None), ("fp16", 2056, 8192, 4096, None),
                                  ("bf16", 4096, 4100, 4096, None), ("bf16", 4097, 4096, 2048, "full"),
                                  ("fp16", 4104, 4096, 2048, "row")], ids=str)
def test_peeled_edges(dev, case):
    name, M, N, K, bias_kind = case
    dtype = {"bf16": torch.bfloat16, "fp16": torch.float16}[name]
    g = gen(M + N)
    a, b = rand((M, K), dtype, g), rand((K, N), dtype, g)
    info = mb.kernels.plan(a, b)
    assert info["tile"][:2] == (256, 256) and info["grid"][0] == 256, info
    mm, nn = M - M % 256, N - N % 256
    if bias_kind is None:
        got = mb.matmul(_to(a, dev), _to(b, dev)).cpu()
        ref_kw = {}
    else:
        bias = rand((M, N) if bias_kind == "full" else (N,), dtype, g)
        got = mb.addmm(_to(bias, dev), _to(a, dev), _to(b, dev), beta=0.5, alpha=2.0).cpu()
        ref_kw = {"bias": bias, "beta": 0.5, "alpha": 2.0}
    # whole rows on both sides of the core / strip boundary, and the last row
    for r in sorted({0, mm - 1, min(mm, M - 1), M - 1}):
        kw = dict(ref_kw)
        if bias_kind == "full":
            kw["bias"] = ref_kw["bias"][r:r + 1]
        assert_parity(got[r:r + 1], a[r:r + 1], b, tag=f"peel {case} row {r}", **kw)
    if nn < N:   # the column strip on sampled rows
        kw = dict(ref_kw)
        if bias_kind is not None:
            kw["bias"] = ref_kw["bias"][..., nn:] if bias_kind == "row" else ref_kw["bias"][:, nn:]
        assert_parity(got[:, nn:], a, b[:, nn:], tag=f"peel {case} columns", **kw)


@pytest.mark.parametrize("case", [("bf16", 4097, 4097, 4097, None, 0), ("fp16", 4096, 4100, 4099, "row", 0),
                                  ("bf16", 4100, 4096, 4097, None, 1), ("bf16", 4097, 4097, 4097, "full", 0)],
                         ids=str)
def test_packed_peel(dev, case):
    """Products whose operands are both copied (odd K, a column-sliced B) and whose M or N ends
    1..16 past a multiple of 256: A and B are copied first (K zero-padded to a stage, B's last
    columns also K-contiguous), then the core runs whole 256 x 256 tiles on the copies and the
    strips the streaming GEMV.  Every element is checked (the oracle on spread rows pins a
    float64 product of the whole output)."""
    name, M, N, K, bias_kind, b_slice = case
    dtype = {"bf16": torch.bfloat16, "fp16": torch.float16}[name]
    g = gen(M + N + K)
    a = rand((M, K), dtype, g).to(dev)
    b = rand((K, N + b_slice), dtype, g).to(dev)[:, :N]
    info = mb.kernels.plan(a, b)
    assert info["tile"][:2] == (256, 256) and info["grid"][0] == 256, info
    if bias_kind is None:
        got = mb.matmul(a, b)
        assert_parity_full(got, a, b, rows=16, tag=f"packed peel {case}")
    else:
        bias = rand((M, N) if bias_kind == "full" else (N,), dtype, g).to(dev)
        got = mb.addmm(bias, a, b, beta=0.5, alpha=2.0)
        assert_parity_full(got, a, b, bias=bias, beta=0.5, alpha=2.0, rows=16, tag=f"packed peel {case}")


# ---- small generic tiles (16 x 16 / 32 x 32, no K slices) -------------------------------------

@pytest.mark.parametrize("dtype", [torch.int16, torch.int32, torch.int64], ids=str)
@pytest.mark.parametrize("shape", [(256, 256, 256), (250, 270, 333), (500, 520, 700), (96, 4096, 1024)], ids=str)
@pytest.mark.parametrize("layout", ["rr", "cc"])
def test_int_full_range_small_tiles(dev, dtype, shape, layout):
    """Full-range integer operands on the generic kernel's 16 x 16 and 32 x 32 tiles (products
    whose 64 x 64 tiles would leave CUs idle and whose K is short): wraparound modulo 2^bits,
    ragged tile edges, both operand orders, the fused integer epilogue and a batch."""
    M, N, K = shape
    d = mb.kernels.plan(torch.empty(M, K, dtype=dtype, device=dev), torch.empty(K, N, dtype=dtype, device=dev))
    assert d["family"] == "generic" and d["tile"][0] in (16, 32) and d["split_k"] == 1, d
    g = gen(91)
    info = torch.iinfo(dtype)
    def full(shape):
        return torch.randint(info.min, info.max, shape, generator=g, dtype=torch.int64).to(dtype)
    a = full((M, K)) if layout[0] == "r" else full((K, M)).t()
    b = full((K, N)) if layout[1] == "r" else full((N, K)).t()
    got = mb.matmul(_to(a, dev), _to(b, dev))
    assert_parity(got, a, b, tag=f"{dtype} {shape} {layout}")
    bias = full((N,))
    got = mb.addmm(bias.to(dev), _to(a, dev), _to(b, dev), beta=-3, alpha=7)
    assert_parity(got, a, b, bias=bias, beta=-3, alpha=7, tag=f"{dtype} addmm {shape} {layout}")
    ab, bb = full((3, M // 2, K)), full((3, K, N // 2))
    got = mb.bmm(ab.to(dev), bb.to(dev))
    assert_parity(got, ab, bb, tag=f"{dtype} bmm {shape}")


# ---- complex64 GEMV on the workgroup-wide row stream (k_cdot_wg, conj as signs) ----------------

@pytest.mark.parametrize("conj", ["none", "a", "b", "ab"])
@pytest.mark.parametrize("shape", [(8192, 8192), (1001, 2048), (3, 512), (4096, 4095), (1, 512)], ids=str)
def test_complex64_gemv_streaming(dev, shape, conj):
    M, K = shape
    g = gen(M + K)
    a = rand((M, K), torch.complex64, g)
    x = rand((K,), torch.complex64, g)
    A, X = a.to(dev), x.to(dev)
    if "a" in conj:
        a, A = a.conj(), A.conj()
    if "b" in conj:
        x, X = x.conj(), X.conj()
    info = mb.kernels.plan(A.resolve_conj(), X.resolve_conj()[:, None])
    if K % 2 == 0:   # the streaming kernel reads 16-byte chunks (two complex elements) of a row
        assert info["family"] == "gemv_dot" and info["tile"][0] == 1 and info["tile"][2] == 1, info
    got = mb.matmul(A, X)
    assert got.shape == (M,)
    assert_parity(got[:, None], a, x[:, None], tag=f"complex gemv {shape} conj={conj}")
    out = torch.empty(M, dtype=torch.complex64, device=dev)
    mb.matmul(A, X, out=out)
    assert torch.equal(out.cpu(), got.cpu())


# ---- deep-K products on the streaming 64 x 64 schedule (K slices on a 1-D grid) ------------------

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", [(128, 128, 65536), (100, 200, 20000), (256, 192, 16448), (2, 96, 128, 24576)],
                         ids=str)
@pytest.mark.parametrize("layout", ["rr", "rc", "cr", "cc"])
def test_deep_k(dev, dtype, shape, layout):
    """Deep-K products: ragged tile edges, a K that ends inside a stage, a batch; every operand
    layout; the fused epilogue on the row-major case."""
    Bb = shape[0] if len(shape) == 4 else None
    M, N, K = shape[-3:]
    g = gen(M + N + K)
    lead = (Bb,) if Bb else ()
    a = rand(lead + (M, K), dtype, g) if layout[0] == "r" else rand(lead + (K, M), dtype, g).transpose(-2, -1)
    b = rand(lead + (K, N), dtype, g) if layout[1] == "r" else rand(lead + (N, K), dtype, g).transpose(-2, -1)
    ad, bd = _to(a, dev), _to(b, dev)
    p = mb.kernels.plan(ad, bd)
    assert p["tile"][5] == 3 and p["split_k"] > 1, p
    got = mb.bmm(ad, bd) if Bb else mb.matmul(ad, bd)
    assert_parity_full(got, ad, bd, rows=8, tag=f"deep-K {dtype} {shape} {layout}")
    if layout == "rr" and not Bb:
        bias = rand((N,), dtype, g).to(dev)
        got = mb.addmm(bias, ad, bd, beta=0.5, alpha=-2.0)
        assert_parity_full(got, ad, bd, bias=bias, beta=0.5, alpha=-2.0, rows=8, tag=f"deep-K addmm {dtype} {shape}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("case", ["natural", "kcontig", "six", "xw", "bmm", "addmm"])
def test_dotx(dev, dtype, case):
    """k_dotx (4 x 8 tile: up to 8 vectors against a K-contiguous matrix, the whole K in one
    workgroup): natural 8-wide vector rows and K-contiguous vectors read in place, 6 vectors
    copied K-contiguous, the transposed form X @ W^T, a batch, the fused epilogue; a partial
    row quad and group, and K ending inside a wave's piece, inside a 128-k chunk row and at a
    wave boundary."""
    g = gen({"natural": 1, "kcontig": 2, "six": 3, "xw": 4, "bmm": 5, "addmm": 6}[case])
    force = {"tile": (4, 8, 64)}
    if case == "natural":
        a, b = rand((2051, 5000), dtype, g), rand((5000, 8), dtype, g)
    elif case == "kcontig":
        a, b = rand((2048, 2056), dtype, g), rand((8, 2056), dtype, g).t()
    elif case == "six":
        a, b = rand((3000, 16384), dtype, g), rand((16384, 6), dtype, g)
    elif case == "xw":
        a, b = rand((8, 4096), dtype, g), rand((2100, 4096), dtype, g).t()
    elif case == "bmm":
        a, b = rand((8, 2048, 3072), dtype, g), rand((8, 3072, 8), dtype, g)
        force = {}
    else:   # 4096 row quads: 256 groups, picked without a tile request
        a, b = rand((16384, 4096), dtype, g), rand((4096, 8), dtype, g)
        force = {}
    ad, bd = _to(a, dev), _to(b, dev)
    p = mb.kernels.plan(ad, bd, **force)
    assert p["family"] == "mfma" and p["tile"][:2] == (4, 8) and p["split_k"] == 1, p
    assert p["workspace_bytes"] == (16384 * 6 * 2 if case == "six" else 0), p
    tag = f"dotx {dtype} {case}"
    if case == "bmm":
        got = mb.bmm(ad, bd)
    elif case == "addmm":
        bias = rand((8,), dtype, g).to(dev)
        got = mb.addmm(bias, ad, bd, beta=0.5, alpha=-2.0)
        assert_parity_full(got, ad, bd, bias=bias, beta=0.5, alpha=-2.0, rows=16, tag=tag)
        return
    else:
        got = mb.matmul(ad, bd, **force)
    assert_parity_full(got, ad, bd, rows=16, tag=tag)
    again = mb.bmm(ad, bd) if case == "bmm" else mb.matmul(ad, bd, **force)
    assert torch.equal(got, again), f"{tag}: repeated call differs"


# ---- chained batch entries (short-K batched products) -----------------------------------

@pytest.mark.parametrize("case", [
    (torch.bfloat16, 96, 512, 512, 64, (64, 128), False, None),
    (torch.float16, 160, 384, 640, 40, (128, 64), False, None),       # K edge inside the stage
    (torch.bfloat16, 256, 256, 256, 64, (64, 64), True, None),        # broadcast B (stride 0)
    (torch.bfloat16, 403, 130, 200, 64, (64, 128), False, None),      # ragged tiles, ragged z
    (torch.bfloat16, 96, 512, 512, 64, (64, 128), False, (0.5, 2.0)),  # fused epilogue, row bias
    (torch.float16, 160, 384, 640, 40, (128, 64), False, (1.0, 1.0)),
    (torch.bfloat16, 64, 1024, 1024, 128, (64, 128), False, None),   # two stages per entry
    (torch.float16, 96, 512, 384, 200, (128, 64), False, None),       # four stages, K edge
    (torch.float16, 96, 512, 512, 192, (64, 64), False, (1.0, 0.0)),  # three stages, alpha 0
    (torch.bfloat16, 100, 512, 512, 256, (64, 64), True, (0.5, 2.0)),
], ids=str)
def test_chained_batch_entries(dev, case):
    """A short K slice (one to four stages) over many batch entries runs on fewer z-blocks,
    each workgroup streaming the stages of its entries through two LDS buffers (the next
    entry's first stage loads during the current entry's last stage and epilogue).  Checked
    through the C ABI on every entry (the oracle on the first and last, the oracle-pinned fp64
    GPU product on all), with a K edge, ragged tile and z ranges, a stride-0 B and a fused
    epilogue (16-bit tiles: the 8-bit ones do not chain)."""
    from metalblas_amd import _lib
    dtype, Bb, M, N, K, tile, bcast, epi = case
    g = gen(Bb + K)
    a = rand((Bb, M, K), dtype, g).to(dev)
    b = rand((1 if bcast else Bb, K, N), dtype, g).to(dev)
    bv = b.expand(Bb, K, N) if bcast else b
    c = torch.empty(Bb, M, N, dtype=dtype, device=dev)
    kw = {}
    bias = None
    if epi is not None:
        beta, alpha = epi
        bias = rand((N,), dtype, g).to(dev)
        kw = dict(epilogue=(beta, alpha, beta != 0, alpha != 0))
    d = _lib.make_desc(dtype, Bb, M, N, K, (a, K, 1, M * K), (b, N, 1, 0 if bcast else K * N),
                       (c, N, 1, M * N), (bias, 0, 1, 0) if bias is not None else None, tile=tile, **kw)
    p = _lib.plan(d)
    assert tuple(p.tile[:2]) == tile and p.split_k == 1, tuple(p.tile)
    assert 0 < p.grid[2] < Bb, f"not chained: grid {tuple(p.grid)}"
    _lib.run(d, dev)
    if epi is None:
        assert_parity_full(c, a, bv, rows=8, tag=f"chained {case}")
    else:
        assert_parity_full(c, a, bv, bias=bias.expand(Bb, M, N), beta=epi[0], alpha=epi[1], rows=8,
                           tag=f"chained {case}")
