// Matrix-core GEMM family for gfx950 (kernel template; instantiated per dtype in
// gemm_mfma_<dtype>.hip) (CDNA4): bf16 / fp16 / fp32 / int8 / uint8.
//
// Replaces the reference's cooperative-tensor and simdgroup GEMMs (shaders/mpp_tensor.h:58-142,
// shaders/mpp_gemm.h:150-427, shaders/simd_gemm.h:153-300, shaders/splitk.h:21-65,
// shaders/int_gemm.h:41-154 for int8/uint8) with one wave64 MFMA design:
//
//   * Block tile BM x BN, wave grid WM x WN (64*WM*WN threads); each wave owns a
//     (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks.
//   * K advances 128 bytes per stage (64 bf16/fp16, 32 fp32, 128 int8).  Both operands are
//     staged in LDS K-major: one 128-byte row per M (or N) index, 8 chunks of 16 bytes, the
//     chunk index XOR-swizzled by (row & 7) ^ ((row >> 3) & 7) so that the 16-byte fragment
//     reads (32 consecutive rows, one chunk) and the transposing writes (rows 8 apart) are
//     both free of bank conflicts.
//   * Operands contiguous along K are copied chunk by chunk.  Operands contiguous along M/N
//     (row-major B, column-major A) are transposed on the way in: each thread loads an
//     E x E element block (E = 16 / element size) with E 16-byte loads and writes E 16-byte
//     K-major chunks; no LDS transpose reads are needed.
//   * Two LDS stages (double buffer) with one barrier per K step; the next stage's global
//     loads are issued before the MFMAs of the current stage.
//   * The MFMA computes C^T = B^T A^T (B tile as the instruction's A operand) so that each
//     lane ends with 4 consecutive output columns of one row: 4-element vector stores.
//   * Fused epilogue alpha*acc + beta*bias (shaders/mb_epi.h:16-26), optional split-K that
//     writes fp32/int32 partial planes summed by a deterministic reduction (no atomics),
//     batched via grid z with per-operand batch strides (stride 0 = broadcast), and an
//     XCD-aware, grouped tile order (the reference's SWIZZLE_LOG idea,
//     shaders/mpp_tensor.h:94-99) so that tiles sharing A rows / B columns run on the
//     same XCD's L2.
#pragma once

#include "launch.hpp"

namespace mb {

namespace mfma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// ---- per-dtype MFMA policy ------------------------------------------------------------
// mma(acc, a, b): acc += a_frag x b_frag for one 16-byte chunk per lane.
template <class T> struct Pol;

template <> struct Pol<bf16_t> {
    using Acc = f32x16;
    static constexpr int ES = 2;
    __device__ static __forceinline__ void mma(Acc &c, uint4 a, uint4 b) {
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};
template <> struct Pol<f16_t> {
    using Acc = f32x16;
    static constexpr int ES = 2;
    __device__ static __forceinline__ void mma(Acc &c, uint4 a, uint4 b) {
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};
template <> struct Pol<float> {
    using Acc = f32x16;
    static constexpr int ES = 4;
    __device__ static __forceinline__ void mma(Acc &c, uint4 a, uint4 b) {
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
    }
};
// int8 and uint8 share the signed i8 MFMA: a byte b read as signed equals b modulo 2^8, so
// the int32 sums agree with the unsigned ones modulo 2^8, and the output keeps 8 bits.
template <> struct Pol<int8_t> {
    using Acc = i32x16;
    static constexpr int ES = 1;
    __device__ static __forceinline__ void mma(Acc &c, uint4 a, uint4 b) {
        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a),
                                                  __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
    }
};
template <> struct Pol<uint8_t> : Pol<int8_t> {};

__device__ __forceinline__ float acc_elem_f(const f32x16 &c, int r) { return c[r]; }

// acc element -> Tr<T>::acc
template <class T, class Acc> __device__ __forceinline__ typename Tr<T>::acc acc_get(const Acc &c, int r) {
    if constexpr (Tr<T>::is_int) return (uint32_t)c[r];
    else return c[r];
}

__device__ __forceinline__ int lds_swz(int row) { return (row & 7) ^ ((row >> 3) & 7); }

// E x E transpose of element blocks held as E 16-byte vectors (E = 16 / element size).
template <int ES> __device__ __forceinline__ void transpose_block(uint4 (&v)[16 / ES]) {
    constexpr int E = 16 / ES;
    if constexpr (ES == 4) {
        uint32_t m[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            m[i][0] = v[i].x; m[i][1] = v[i].y; m[i][2] = v[i].z; m[i][3] = v[i].w;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = make_uint4(m[0][j], m[1][j], m[2][j], m[3][j]);
    } else if constexpr (ES == 2) {
        // in[i] holds (row i, cols 0..7); out[j] = (col j, rows 0..7)
        uint32_t w[8][4];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            w[i][0] = v[i].x; w[i][1] = v[i].y; w[i][2] = v[i].z; w[i][3] = v[i].w;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t o[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                // elements (row 2p, col j) and (row 2p+1, col j)
                const uint32_t lo = w[2 * p][j >> 1], hi = w[2 * p + 1][j >> 1];
                o[p] = (j & 1) ? __builtin_amdgcn_perm(hi, lo, 0x07060302u)
                               : __builtin_amdgcn_perm(hi, lo, 0x05040100u);
            }
            v[j] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    } else {
        // 16 x 16 bytes
        uint8_t b[16][16];
#pragma unroll
        for (int i = 0; i < E; ++i) __builtin_memcpy(b[i], &v[i], 16);
        uint8_t t[16][16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int j = 0; j < 16; ++j) t[j][i] = b[i][j];
#pragma unroll
        for (int j = 0; j < E; ++j) __builtin_memcpy(&v[j], t[j], 16);
    }
}

// Loader of one operand tile (ROWS x 128 bytes of K) into K-major swizzled LDS.
//   KC: operand contiguous along K: element (row, k) at p[row*ld + k]
//   else contiguous along rows:      element (row, k) at p[k*ld + row]
template <class T, int ROWS, int NT, bool KC> struct TileLoader {
    static constexpr int ES = sizeof(T);
    static constexpr int E = 16 / ES;        // elements per 16-byte chunk
    static constexpr int CH = ROWS * 8;      // 16-byte chunks per stage
    static constexpr int NLOAD = (CH + NT - 1) / NT;   // 16-byte loads per thread
    static constexpr int NBLK = (ROWS / E) * 8;         // transpose blocks (non-KC)
    static constexpr int BPT = (NBLK + NT - 1) / NT;   // blocks per thread (non-KC)
    uint4 r[KC ? NLOAD : BPT * E];

    __device__ __forceinline__ void load(const T *p, int64_t ld, int row0, int rows_lim, int k0, int k_lim,
                                         int tid) {
        if constexpr (KC) {
#pragma unroll
            for (int i = 0; i < NLOAD; ++i) {
                const int c = tid + i * NT;
                const int row = c >> 3, kc = c & 7;
                const int gr = row0 + row, gk = k0 + kc * E;
                uint4 v = make_uint4(0, 0, 0, 0);
                if ((CH % NT == 0 || c < CH) && gr < rows_lim && gk < k_lim)
                    v = *(const uint4 *)(p + gr * ld + gk);
                r[i] = v;
            }
        } else {
#pragma unroll
            for (int bi = 0; bi < BPT; ++bi) {
                const int blk = tid + bi * NT;
                const int rb = blk % (ROWS / E), kb = blk / (ROWS / E);
                const int gr = row0 + rb * E;
#pragma unroll
                for (int i = 0; i < E; ++i) {
                    const int gk = k0 + kb * E + i;
                    uint4 v = make_uint4(0, 0, 0, 0);
                    if ((NBLK % NT == 0 || blk < NBLK) && gr < rows_lim && gk < k_lim)
                        v = *(const uint4 *)(p + gk * ld + gr);
                    r[bi * E + i] = v;
                }
            }
        }
    }

    __device__ __forceinline__ void store(char *lds, int tid) {
        if constexpr (KC) {
#pragma unroll
            for (int i = 0; i < NLOAD; ++i) {
                const int c = tid + i * NT;
                if (CH % NT != 0 && c >= CH) continue;
                const int row = c >> 3, kc = c & 7;
                *(uint4 *)(lds + row * 128 + ((kc ^ lds_swz(row)) << 4)) = r[i];
            }
        } else {
#pragma unroll
            for (int bi = 0; bi < BPT; ++bi) {
                const int blk = tid + bi * NT;
                if (NBLK % NT != 0 && blk >= NBLK) continue;
                const int rb = blk % (ROWS / E), kb = blk / (ROWS / E);
                uint4 blkv[E];
#pragma unroll
                for (int i = 0; i < E; ++i) blkv[i] = r[bi * E + i];
                transpose_block<ES>(blkv);
#pragma unroll
                for (int j = 0; j < E; ++j) {
                    const int row = rb * E + j;
                    *(uint4 *)(lds + row * 128 + ((kb ^ lds_swz(row)) << 4)) = blkv[j];
                }
            }
        }
    }
};

// Logical tile index from the hardware workgroup id: XCD-contiguous ranges, then groups of
// 2^swz tile rows walked column by column.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int swz, int &tm, int &tn) {
    const int n = tiles_m * tiles_n;
    if (n >= 16) {
        const int xcd = pid & 7, idx = pid >> 3;
        const int base = n >> 3, rem = n & 7;
        pid = xcd * base + min(xcd, rem) + idx;
    }
    const int G = 1 << swz;
    const int width = G * tiles_n;
    const int grp = pid / width;
    const int first_m = grp * G;
    const int gsz = min(tiles_m - first_m, G);
    const int in = pid - grp * width;
    tm = first_m + in % gsz;
    tn = in / gsz;
}

template <class T, int BM, int BN, int WM, int WN, bool A_KC, bool B_KC>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_mfma(GemmArgs g) {
    using P = Pol<T>;
    using Acc = typename P::Acc;
    constexpr int NT = 64 * WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN;   // wave sub-tile
    constexpr int TM = WTM / 32, TN = WTN / 32;   // 32x32 blocks per wave
    constexpr int E = 16 / P::ES;                 // elements per chunk
    constexpr int BK = 8 * E;                     // elements of K per stage
    constexpr int STAGE = (BM + BN) * 128;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32x32 block");

    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int tiles_m = cdiv(g.M, BM), tiles_n = cdiv(g.N, BN);
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, g.swz, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);
    const int nk = cdiv(kend - kbeg, BK);

    // lda / ldb: the stride that is not 1
    const int64_t lda = A_KC ? g.a_rs : g.a_cs;
    const int64_t ldb = B_KC ? g.b_cs : g.b_rs;

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const T *Ab = (const T *)g.a + bz * g.a_bs;
        const T *Bb = (const T *)g.b + bz * g.b_bs;

        TileLoader<T, BM, NT, A_KC> la;
        TileLoader<T, BN, NT, B_KC> lb;

        Acc acc[TN][TM];
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

        if (nk > 0) {
            la.load(Ab, lda, m0, g.M, kbeg, kend, tid);
            lb.load(Bb, ldb, n0, g.N, kbeg, kend, tid);
            la.store(smem, tid);
            lb.store(smem + BM * 128, tid);
        }
        __syncthreads();

        for (int kt = 0; kt < nk; ++kt) {
            char *cur = smem + (kt & 1) * STAGE;
            char *nxt = smem + ((kt + 1) & 1) * STAGE;
            const bool more = kt + 1 < nk;
            if (more) {
                const int k0 = kbeg + (kt + 1) * BK;
                la.load(Ab, lda, m0, g.M, k0, kend, tid);
                lb.load(Bb, ldb, n0, g.N, k0, kend, tid);
            }
            const char *As = cur;
            const char *Bs = cur + BM * 128;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int chunk = 2 * s + (lane >> 5);
                uint4 fa[TM], fb[TN];
#pragma unroll
                for (int j = 0; j < TM; ++j) {
                    const int row = wm * WTM + j * 32 + (lane & 31);
                    fa[j] = *(const uint4 *)(As + row * 128 + ((chunk ^ lds_swz(row)) << 4));
                }
#pragma unroll
                for (int i = 0; i < TN; ++i) {
                    const int row = wn * WTN + i * 32 + (lane & 31);
                    fb[i] = *(const uint4 *)(Bs + row * 128 + ((chunk ^ lds_swz(row)) << 4));
                }
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) P::mma(acc[i][j], fb[i], fa[j]);
            }
            if (more) {
                la.store(nxt, tid);
                lb.store(nxt + BM * 128, tid);
            }
            __syncthreads();
        }

        // ---- epilogue: lane holds C[m][n0' + 8*(r/4) + 4*(lane/32) + r%4] for r < 16 ----
        const int mrow = lane & 31;
        const int nsub = 4 * (lane >> 5);
        T *Cb = (T *)g.c + bz * g.c_bs;
        const bool split = g.splits > 1 || g.planes;
        using AccT = typename Tr<T>::acc;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int gm = m0 + wm * WTM + j * 32 + mrow;
                if (gm >= g.M) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int gn = n0 + wn * WTN + i * 32 + 8 * q + nsub;
                    if (split) {
                        AccT *ws = (AccT *)g.ws + (((int64_t)ks * g.batch + bz) * g.M + gm) * g.N;
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (gn + r < g.N) ws[gn + r] = acc_get<T>(acc[i][j], 4 * q + r);
                        continue;
                    }
                    if (g.vec_ok && !g.epilogue && gn + 3 < g.N) {
                        // 4 consecutive outputs: one vector store (alignment checked by the planner)
                        T o[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[r] = Tr<T>::down(acc_get<T>(acc[i][j], 4 * q + r));
                        T *dst = Cb + gm * g.c_rs + gn;
                        if constexpr (sizeof(T) == 2) {
                            uint2 u;
                            __builtin_memcpy(&u, o, 8);
                            *(uint2 *)dst = u;
                        } else if constexpr (sizeof(T) == 4) {
                            uint4 u;
                            __builtin_memcpy(&u, o, 16);
                            *(uint4 *)dst = u;
                        } else {
                            uint32_t u;
                            __builtin_memcpy(&u, o, 4);
                            *(uint32_t *)dst = u;
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int n = gn + r;
                            if (n < g.N)
                                store_out<T>(g, Cb + gm * g.c_rs + n * g.c_cs, acc_get<T>(acc[i][j], 4 * q + r),
                                             bz * g.bias_bs + gm * g.bias_rs + n * g.bias_cs);
                        }
                    }
                }
            }
    }
}

template <class T, int BM, int BN, int WM, int WN>
hipError_t launch_tile(bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    dim3 block(64 * WM * WN);
    if (a_kc && b_kc)
        hipLaunchKernelGGL((k_gemm_mfma<T, BM, BN, WM, WN, true, true>), grid, block, 0, st, g);
    else if (a_kc && !b_kc)
        hipLaunchKernelGGL((k_gemm_mfma<T, BM, BN, WM, WN, true, false>), grid, block, 0, st, g);
    else if (!a_kc && b_kc)
        hipLaunchKernelGGL((k_gemm_mfma<T, BM, BN, WM, WN, false, true>), grid, block, 0, st, g);
    else
        hipLaunchKernelGGL((k_gemm_mfma<T, BM, BN, WM, WN, false, false>), grid, block, 0, st, g);
    return hipGetLastError();
}

template <class T>
hipError_t launch_typed(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
#define MB_TILE(BM, BN, WM, WN) \
    if (t.bm == BM && t.bn == BN && t.wm == WM && t.wn == WN) return launch_tile<T, BM, BN, WM, WN>(a_kc, b_kc, g, grid, st);
    MB_TILE(256, 256, 2, 2)
    MB_TILE(256, 128, 2, 2)
    MB_TILE(128, 256, 2, 2)
    MB_TILE(128, 128, 2, 2)
    MB_TILE(128, 64, 2, 2)
    MB_TILE(64, 128, 2, 2)
    MB_TILE(64, 64, 2, 2)
    MB_TILE(32, 32, 1, 1)
#undef MB_TILE
    return hipErrorInvalidValue;
}

}  // namespace mfma

}  // namespace mb
