// Internal launcher interface between the C ABI / planner (mb_api.hip) and the kernel
// translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mb_types.hpp"

namespace mb {

// dtype codes (same values as mb_dtype in include/metalblas_amd.h)
enum Dt : int { F32 = 0, F16, BF16, C64, C32, I8, U8, I16, I32, I64, DT_COUNT };

inline int dtype_size(int dt) {
    switch (dt) {
        case F32: return 4;
        case F16: case BF16: return 2;
        case C64: return 8;
        case C32: return 4;
        case I8: case U8: return 1;
        case I16: return 2;
        case I32: return 4;
        case I64: return 8;
    }
    return 0;
}
// bytes of one accumulator element (split-K partial planes)
inline int acc_size(int dt) {
    switch (dt) {
        case C64: case C32: case I64: return 8;
        default: return 4;
    }
}

// Invoke f.template operator()<T>() with the storage type of dtype `dt`.
template <class F> inline hipError_t with_dtype(int dt, F &&f) {
    switch (dt) {
        case F32: return f.template operator()<float>();
        case F16: return f.template operator()<f16_t>();
        case BF16: return f.template operator()<bf16_t>();
        case C64: return f.template operator()<c64_t>();
        case C32: return f.template operator()<c32_t>();
        case I8: return f.template operator()<int8_t>();
        case U8: return f.template operator()<uint8_t>();
        case I16: return f.template operator()<int16_t>();
        case I32: return f.template operator()<int32_t>();
        case I64: return f.template operator()<int64_t>();
    }
    return hipErrorInvalidValue;
}

// ---- GEMV families --------------------------------------------------------------------
// Y(i, v) = sum_k Mat(i, k) * X(k, v)   for i < rows, v < nv   (one problem per batch index)
//   dot  family: Mat(i, k) at mat[i*mat_ld + k]     (rows contiguous along K)
//   axpy family: Mat(i, k) at mat[k*mat_ld + i]     (rows of the stored matrix run along i)
struct GemvArgs {
    const void *mat;
    int64_t mat_ld, mat_bs;
    const void *x;
    int64_t x_ks, x_vs, x_bs;
    void *y;
    int64_t y_is, y_vs, y_bs;
    const void *bias;
    int64_t bias_is, bias_vs, bias_bs;
    void *ws;   // axpy split partials: acc-typed [splits][batch][nv][rows]
    int32_t rows, K, nv, batch;
    int32_t conj_mat, conj_x;
    int32_t epilogue, beta_nz, alpha_nz;
    int32_t vec_ok;
    int32_t splits, k_chunk;
    int32_t grid_cap;   // persistent kernels: at most this many workgroups (0 = no cap)
    int32_t x_row;      // dot family: X stored with its nv values contiguous per k
    EpiScalars s;
};

struct LaunchShape {
    dim3 grid, block;
};

// Operand copy into a loader-friendly layout: dst(b, r, c) = src(b, r, c) for r < rows,
// c < cols, and 0 in the padding up to rows_p x cols_p.  Strides are in elements.
struct PackArgs {
    const void *src;
    void *dst;
    int64_t s_rs, s_cs, s_bs;
    int64_t d_rs, d_cs, d_bs;
    int32_t rows, cols, rows_p, cols_p, batch;
    int32_t contig_cols;   // 1: destination contiguous along columns (d_cs == 1), else rows
    int32_t es;            // element bytes: 1, 2, 4 or 8
};

// Complex product as a real one: C (M x N complex) = A (M x K complex) @ B (K x N complex) is
// the real product Chat (M x 2N) = Ahat (M x 2K) @ Bhat (2K x 2N), where Ahat is A's
// interleaved (re, im) storage read as a real matrix and Bhat expands each element b of B
// into the 2 x 2 block [[re b, s_b im b], [-s_a s_b im b, s_a re b]] (s = -1 for a
// conjugated operand).  Bhat is written K-contiguous: element (k', n') at dst[n' * ld + k'],
// zero-padded for k' in [2K, ld).
struct CplxExpandArgs {
    const void *b;
    int64_t b_rs, b_cs, b_bs;   // complex element strides of B
    void *dst;
    int64_t ld, d_bs;           // real element strides of Bhat
    int32_t K, N, batch;
    int32_t neg_a, neg_b;       // conj(A), conj(B)
    int32_t half;               // 1: complex32 (fp16 parts), 0: complex64 (fp32 parts)
};

// gemm_generic.hip
hipError_t launch_cplx_expand(const CplxExpandArgs &a, hipStream_t st);
hipError_t launch_pack(const PackArgs &a, hipStream_t st);
// two operand copies in one launch when both are 16-bit row copies (else two launches)
hipError_t launch_pack2(const PackArgs &a0, const PackArgs &a1, hipStream_t st);
// bt: the square output tile, 64, 32 or 16
hipError_t launch_generic(int dt, int bt, const GemmArgs &g, hipStream_t st, LaunchShape *shape);
hipError_t launch_fill(int dt, const GemmArgs &g, hipStream_t st);
hipError_t launch_splitk_reduce(int dt, const GemmArgs &g, hipStream_t st);
namespace m16 {
// whether k_thin_dot can address 16 rows of A plus a K slice with 31-bit buffer offsets
bool thin_dot_offsets_fit(const GemmArgs &g);
// whether k_thin_dot4 can address the whole matrix and 16 vectors with 31-bit buffer offsets
bool thin_dot4_offsets_fit(const GemmArgs &g);
constexpr int kThinDot4Chunk = 4096;   // K per slice of k_thin_dot4 (4 waves x 8 loads x 128 k)
// k_dotx (up to 8 vectors, the whole K in one workgroup): 16-byte loads per lane per row quad,
// K per wave, row quads per workgroup group, waves per workgroup at most
constexpr int kDotxU = 8, kDotxKW = 128 * kDotxU, kDotxQG = 16, kDotxMaxWaves = 16;
// waves of the k_dotx workgroup for a K (a power of two covering K / 1024)
int dotx_waves(int64_t K);
// whether k_dotx addresses the matrix and the vector block with 31-bit buffer offsets
bool dotx_offsets_fit(const GemmArgs &g, bool xkc);
}  // namespace m16

// gemv.hip
int gemv_nv_bucket(int nv);   // template NV used for a given number of vectors
hipError_t launch_gemv_dot(int dt, const GemvArgs &g, hipStream_t st, LaunchShape *shape);
hipError_t launch_gemv_axpy(int dt, const GemvArgs &g, hipStream_t st, LaunchShape *shape);
int gemv_axpy_vec(int dt, int nv);   // elements per lane of the vector path

// gemv_fast.hip: streaming float kernels (16-byte aligned operands, K or rows multiple of
// the 16-byte vector width)
bool gemv_fast_dtype(int dt);
int gemv_fast_vec(int dt);
// columns one workgroup of the fast axpy kernel covers when it uses column bands (nv == 1),
// else 0; the band narrows for matrices with fewer columns
int gemv_axpy_band_cols(int dt, int nv, int64_t rows);
hipError_t launch_gemv_dot_fast(int dt, const GemvArgs &g, hipStream_t st, LaunchShape *shape);
hipError_t launch_gemv_axpy_fast(int dt, const GemvArgs &g, hipStream_t st, LaunchShape *shape);

// gemm_mfma.hip
struct MfmaTile {
    int bm, bn, wm, wn;   // block tile and wave grid
    int sched = 0;        // 0: interleaved LDS reads / MFMAs per wave; 1: two-group ping-pong;
                          // 2: deep-K streaming ring over a 1-D grid of K slices (64 x 64, bf16 / fp16)
};
bool mfma_supported_dtype(int dt);
int mfma_k_align(int dt);   // elements per 16-byte chunk along K
bool mfma_tile_compiled(int dt, const MfmaTile &t);
int mfma_list_tiles(int dt, MfmaTile *out, int cap);
// a_kc: A contiguous along K (row-major A);  b_kc: B contiguous along K (column-major B)
hipError_t launch_mfma(int dt, const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g,
                       hipStream_t st, LaunchShape *shape);

}  // namespace mb
