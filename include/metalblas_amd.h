/*
 * metalblas_amd.h — C ABI of libmetalblas_hip.so, the gfx950 (MI355X) matmul library.
 *
 * One descriptor-driven entry point (mb_gemm) runs every product the metalblas Python API
 * exposes: C[b] = alpha * op(A[b]) @ op(B[b]) + beta * bias[b], for the full dtype set
 * (fp32/fp16/bf16, complex64/complex32, int8/uint8/int16/int32/int64), any element strides
 * (row-major, column-major, sliced, offset, stride-0 broadcast batches), optional
 * conjugation, and an optional fused epilogue.
 *
 * Conventions
 *   - All pointers are device pointers; strides are in ELEMENTS (a complex element counts once).
 *   - The library never allocates device memory and never synchronises.  Kernels are queued
 *     on the caller's stream (a hipStream_t passed as void*; NULL = the null stream).
 *   - Scratch space (split-K partial planes) is provided by the caller: query the size with
 *     mb_gemm_workspace_bytes() for the same descriptor and pass it in desc->workspace.  One
 *     workspace may serve successive calls on one stream, but a call queues up to several
 *     kernels (a split-K product and its reduction), so calls queued concurrently from several
 *     host threads need distinct workspaces, or a lock held across each mb_gemm() call.
 *   - Return value 0 = success, negative = mb_status (see mb_strerror()).
 *   - Thread-safe.  Mutable global state, each guarded by a mutex: the per-process
 *     device-property cache, the plan cache of mb_gemm() (up to 1024 call signatures), and the
 *     per-device address table of mb_gemm_noalloc()'s static scratch buffer.
 *
 * Reference interfaces this ABI replaces (Isalia20/metalBLAS, file:line):
 *   - the Metal kernel handles assembled by metalblas/kernels.py:76-253 and launched as
 *     fn(*buffers, threads=, group_size=) by metalblas/float_dispatch.py:745-852,897-956,1049-1091,
 *     metalblas/integer_dispatch.py:57-150 and metalblas/complex_dispatch.py:33-144;
 *   - the dims/stride structs those kernels bind (MBTensorDims shaders/mpp_tensor.h:56,
 *     MBGemmDims shaders/mpp_gemm.h:148, MBIntGemmDims shaders/int_gemm.h:39, the batch
 *     int4 (sA,sB,sC,sBias) shaders/mpp_tensor.h:70) and the epilogue buffers
 *     (bias, bstride, beta, alpha) of shaders/mb_epi.h:16-26.
 */
#ifndef METALBLAS_AMD_H
#define METALBLAS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MB_ABI_VERSION 1

/* Element types.  Integer products accumulate with wraparound in 32 bits (64 for int64) and
 * are truncated to the input width, as metalblas/integer_dispatch.py:13-19 specifies.
 * Floating types accumulate in fp32 (metalblas/float_dispatch.py:25-29). */
typedef enum mb_dtype {
    MB_DTYPE_F32 = 0,
    MB_DTYPE_F16 = 1,
    MB_DTYPE_BF16 = 2,
    MB_DTYPE_C64 = 3,   /* interleaved (re, im) float pairs */
    MB_DTYPE_C32 = 4,   /* interleaved (re, im) fp16 pairs (torch.complex32) */
    MB_DTYPE_I8 = 5,
    MB_DTYPE_U8 = 6,
    MB_DTYPE_I16 = 7,
    MB_DTYPE_I32 = 8,
    MB_DTYPE_I64 = 9,
    MB_DTYPE_COUNT = 10
} mb_dtype;

/* Kernel family selection; mirrors backend= of metalblas/float_dispatch.py:802-852. */
typedef enum mb_backend {
    MB_BACKEND_AUTO = 0,     /* planner decides (backend=None / "auto") */
    MB_BACKEND_GEMV = 1,     /* "gemv": matrix-vector family, requires M==1 or N==1 */
    MB_BACKEND_MATRIX = 2,   /* "mpp_tensor": matrix-core tile family, tile=(BM, BN, waves) */
    MB_BACKEND_TILED = 3,    /* "mpp"/"simd": matrix-core family, tile=(BM, BN, BK, WM, WN) */
    MB_BACKEND_GENERIC = 4,  /* element-gather VALU kernel: any strides, any alignment */
    MB_BACKEND_COUNT = 5
} mb_backend;

typedef enum mb_status {
    MB_OK = 0,
    MB_ERR_INVALID_ARG = -1,        /* bad sizes / null pointers / bad strides */
    MB_ERR_UNSUPPORTED_DTYPE = -2,
    MB_ERR_UNSUPPORTED_LAYOUT = -3, /* a forced backend cannot run this layout */
    MB_ERR_WORKSPACE = -4,          /* workspace missing or too small */
    MB_ERR_LAUNCH = -5,             /* hipGetLastError() after a launch */
    MB_ERR_NO_DEVICE = -6,
    MB_ERR_GEMV_SHAPE = -7,         /* backend GEMV with M != 1 and N != 1 */
    MB_ERR_BAD_BACKEND = -8,
    MB_ERR_SCRATCH_LIMIT = -9       /* mb_gemm_noalloc: the product needs more scratch than its
                                       static buffer holds */
} mb_status;

/* A strided (batched) matrix operand.  Element (b, r, c) lives at
 * ptr + b*batch_stride + r*row_stride + c*col_stride. */
typedef struct mb_matrix {
    void *ptr;
    int64_t row_stride;
    int64_t col_stride;
    int64_t batch_stride;
} mb_matrix;

typedef struct mb_gemm_desc {
    int32_t dtype;        /* mb_dtype; A, B, C and bias share it */
    int32_t backend;      /* mb_backend */
    int64_t batch;        /* >= 1 */
    int64_t M, N, K;      /* C is M x N, A is M x K, B is K x N; K == 0 gives beta*bias (or 0) */
    mb_matrix a;          /* read-only */
    mb_matrix b;          /* read-only */
    mb_matrix c;          /* written */
    mb_matrix bias;       /* read only when epilogue && beta_nz; stride 0 broadcasts */
    int32_t conj_a;       /* complex only: use conj(A) */
    int32_t conj_b;       /* complex only: use conj(B) */
    int32_t epilogue;     /* 0: C = A@B;  1: C = alpha*(A@B) + beta*bias (one final rounding) */
    int32_t beta_nz;      /* epilogue: bias term present (bias not read when 0: NaN-safe) */
    int32_t alpha_nz;     /* epilogue: product term present */
    int32_t swizzle_log;  /* tile-order group size 2^swizzle_log; -1 = auto */
    double alpha_re, alpha_im;  /* float / complex scalars (fp32 arithmetic on device) */
    double beta_re, beta_im;
    int64_t alpha_int, beta_int;  /* integer dtypes: taken modulo 2^(accumulator bits) */
    int32_t tile[8];      /* 0-filled = auto; see MB_BACKEND_* for the meaning */
    int32_t split_k;      /* 0 = auto, 1 = off, >1 = number of K slices (matrix-core family) */
    int32_t flags;        /* 0, or MB_FLAG_DRY_RUN; other bits are rejected */
    void *workspace;      /* caller-provided device scratch (see mb_gemm_workspace_bytes) */
    int64_t workspace_bytes;
} mb_gemm_desc;

/* desc->flags: plan the call exactly as mb_gemm() would (through its per-signature plan cache,
 * including METALBLAS_LAUNCH_CACHE=verify) and return MB_OK without queuing any work.  For
 * host-side tests of the planner and the cache: no kernel is launched, so a descriptor's
 * pointers need not be valid device memory. */
#define MB_FLAG_DRY_RUN 1

/* What the planner chose for a descriptor (for tests, the autotuner and reports). */
typedef struct mb_plan_info {
    int32_t family;        /* mb_family */
    int32_t tile[8];       /* family-specific tile parameters */
    int32_t split_k;       /* K slices actually used */
    int32_t swizzle_log;
    int32_t transposed;    /* 1 if computed as C^T = B^T A^T */
    int32_t grid[3];
    int32_t block;
    int64_t workspace_bytes;
} mb_plan_info;

typedef enum mb_family {
    MB_FAMILY_NONE = 0,       /* nothing to compute (empty output) */
    MB_FAMILY_FILL = 1,       /* K == 0: C = beta*bias or 0 */
    MB_FAMILY_GENERIC = 2,    /* LDS-tiled VALU kernel, any layout */
    MB_FAMILY_MFMA = 3,       /* matrix-core GEMM (bf16/fp16/fp32/int8/uint8/complex) */
    MB_FAMILY_GEMV_DOT = 4,   /* matrix rows contiguous along K (gemv_nt-like) */
    MB_FAMILY_GEMV_AXPY = 5   /* matrix rows contiguous along the output dim (gemv_t-like) */
} mb_family;

/* Queue C = alpha*op(A)@op(B) + beta*bias on `stream` (a hipStream_t).
 * Replaces the kernel launches of metalblas/float_dispatch.py:745-852 (matmul),
 * :897-956 (addmm), :1049-1091 (bmm/baddbmm), metalblas/integer_dispatch.py:92-150 and
 * metalblas/complex_dispatch.py:33-144.  Plans are cached per call signature (the descriptor
 * with pointers reduced to null-ness and their low 8 bits, workspace present or absent, current
 * device; up to 1024 signatures, thread-safe): a repeated call skips the planner.
 * METALBLAS_LAUNCH_CACHE=0 disables the cache; =verify replans every hit and aborts on a
 * difference. */
int mb_gemm(const mb_gemm_desc *desc, void *stream);

/* mb_gemm() without a workspace and without any allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The split-K planes, operand copies and complex
 * expansions a product needs run in a static per-device buffer of
 * mb_gemm_noalloc_scratch_bytes() bytes (64 MiB, enough for every benchmark workload) that the
 * library holds on each device it runs on until the process ends; desc->workspace and
 * desc->workspace_bytes are ignored.  The plan is the one mb_gemm() runs with a workspace of
 * mb_gemm_noalloc_scratch_bytes() bytes: the same kernels, hence identical results, for every
 * product whose full plan fits the buffer (mb_gemm_workspace_bytes() <= that size), edge-peeled
 * products included.  A product whose peeled plan would not fit runs unpeeled if that fits;
 * one that needs more scratch than the buffer holds either way returns MB_ERR_SCRATCH_LIMIT and
 * queues nothing.  Calls share the device's buffer: calls that
 * overlap on one device (different streams or host threads) race; calls queued on one stream
 * are ordered and safe.  desc->flags may be 0 or MB_FLAG_DRY_RUN (every entry point rejects
 * other bits with MB_ERR_INVALID_ARG). */
int mb_gemm_noalloc(const mb_gemm_desc *desc, void *stream);

/* Size of mb_gemm_noalloc's static per-device scratch buffer, in bytes. */
int64_t mb_gemm_noalloc_scratch_bytes(void);

/* Bytes of device scratch mb_gemm() needs for this descriptor (0 if none); negative on error.
 * Replaces the pooled split-K partial planes of metalblas/float_dispatch.py:183-192. */
int64_t mb_gemm_workspace_bytes(const mb_gemm_desc *desc);

/* Fill *info with the plan mb_gemm() runs when given the workspace that
 * mb_gemm_workspace_bytes() reports (without it, split-K is dropped).  A bf16/fp16 product
 * that mb_gemm() runs as whole 256 x 256 tiles plus a 1..16-row (column) edge strip reports
 * the tiled core; workspace_bytes is then the largest part's.  Replaces the plan caches/pickers of
 * metalblas/float_dispatch.py:484-505 (_gemm_plan) and :613-655 (_pick_mpp_tensor_tile). */
int mb_plan(const mb_gemm_desc *desc, mb_plan_info *info);

/* Autotune candidates: up to `cap` entries of 8 int32 worth timing for this descriptor;
 * returns the count.  Entry 0 is the static plan (its matrix-core tile, or zeros for a GEMV
 * plan; a tuner runs it without a request).  Each other entry is a request that plans to a
 * different kernel: entries 0-5 go to desc->tile, entry 6 to desc->split_k (0 = the planner's
 * K slices).  The rivals span the kernel families: the other compiled matrix-core tiles, the
 * thin-product kernels (products with at most 32 rows or columns) and other K-slice counts of
 * the static tile.  Replaces metalblas/float_dispatch.py:369-404 (_mpp_tensor_tile_candidates)
 * and the cross-family candidates of :439-481 and :516-542. */
int mb_tile_candidates(const mb_gemm_desc *desc, int32_t *tiles, int cap);

/* Queries.  Replaces metalblas/kernels.py:65-73 (has_metal4) and the chip detection of
 * metalblas/float_dispatch.py:32-51. */
typedef enum mb_query_what {
    MB_QUERY_ABI_VERSION = 0,
    MB_QUERY_HAS_MATRIX_CORES = 1,  /* 1 when the current device is gfx950 */
    MB_QUERY_CU_COUNT = 2,
    MB_QUERY_GFX_ARCH = 3,          /* e.g. 950 */
    MB_QUERY_LDS_BYTES = 4          /* LDS per workgroup available to kernels */
} mb_query_what;
int64_t mb_query(int32_t what);

/* Static message for a status code. */
const char *mb_strerror(int32_t status);

#ifdef __cplusplus
}
#endif

#endif /* METALBLAS_AMD_H */
