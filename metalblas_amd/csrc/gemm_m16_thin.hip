// Thin products on the matrix cores, bf16_t / f16_t: a handful of vectors against a large
// matrix that is streamed from HBM exactly once.
//
//   * k_thin16 (mfma16.hpp), tile 32 x 256 or 32 x 128: the vectors (up to 32) are the rows of
//     A (K-contiguous), the matrix B is N-contiguous; B goes through a 4-deep LDS-direct ring
//     (512- or 256-byte row spans).
//   * k_thin_dot (below), tile 64 x 16: the matrix A is K-contiguous and the vectors are the
//     columns of B (K-contiguous).  The matrix never touches LDS: each wave loads 1 KiB of
//     each of its 16 rows per 512-deep macro step straight into the registers that feed
//     v_mfma_f32_16x16x32 (the row-contiguous stream of the GEMV kernels), double-buffered
//     across macro steps.  Only the 16 x 512 vector
//     slice of a step is staged in LDS, shared by the workgroup's 4 waves.
//
// The planner transposes the other two layout combinations into these two.
#include "mfma16.hpp"

namespace mb {
namespace m16 {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <class T> __device__ __forceinline__ f32x4 mma16x16(uint4 a, uint4 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mma16x16<bf16_t>(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}
template <> __device__ __forceinline__ f32x4 mma16x16<f16_t>(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// 16-byte buffer load; offsets past the resource's 2 GiB range read zeros (the
// offsets used below stay under 2^32)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ uint4 ld_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// C (M x N, N <= 16) = A (M x K, K-contiguous) @ B (K x N, K-contiguous), fp32 accumulation.
// Workgroup: 4 waves x 16 rows of A; grid (ceil(M / 64), K slices, batch).  g.k_chunk is a
// multiple of KS and K a multiple of 8, so a 16-byte chunk is either inside the slice or past
// its end (then it contributes zeros).
//
// v_mfma_f32_16x16x32 takes, in lane l, 8 consecutive k of row l % 16 of its first operand and
// of column l % 16 of its second, for the k group l / 16, and returns D[4 (l / 16) + i][l % 16].
// MFMA j of a step covers k0 + 32 j .. k0 + 32 j + 31.  The first operand is the vector slice (rows n), the second the matrix rows
// (columns m): lane l ends with C[m0 + l % 16][4 (l / 16) + i].
template <class T>
__global__ __launch_bounds__(256) void k_thin_dot(GemmArgs g) {
    constexpr int KS = 512, XP = KS + 8;   // k per macro step; LDS row pitch (conflict-free reads)
    __shared__ __attribute__((aligned(16))) T xs[2][16][XP];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: the resource stays scalar
    const int r = lane & 15, grp = lane >> 4;
    const int m0 = blockIdx.x * 64 + 16 * w;
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);
    const int nsteps = cdiv(kend - kbeg, KS);
    // rows past M repeat row M - 1: their values are never stored
    const int mbase = min(m0, g.M - 1), mrow = min(m0 + r, g.M - 1);
    // byte offset of this lane's row and k group from the wave's first row (the host checks
    // 16 rows + K fit in 31 bits)
    const uint32_t lane_off = (uint32_t)(((int64_t)(mrow - mbase) * g.a_rs + 8 * grp) * sizeof(T));
    uint32_t x_off[4];   // byte offsets of this thread's vector chunks (k from the step start)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        x_off[i] = (uint32_t)(((int64_t)(c >> 6) * g.b_cs + 8 * (c & 63)) * sizeof(T));
    }

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const __amdgpu_buffer_rsrc_t ra = buf_rsrc((const T *)g.a + bz * g.a_bs + (int64_t)mbase * g.a_rs);
        // vector n, K-contiguous: element k at (n * b_cs + k) from the batch's B
        const __amdgpu_buffer_rsrc_t rb = buf_rsrc((const T *)g.b + bz * g.b_bs);

        // this lane's 16 chunks of step st: k = kbeg + st KS + 32 j + 8 grp, so load j reads 64
        // contiguous bytes of each of the wave's 16 rows and the wave's 16 loads cover 1 KiB
        // of every row back to back (the chunk offset rides in the scalar offset: one VGPR
        // addresses all 16 loads)
        auto load_w = [&](int st, uint4 (&dst)[16]) {
            const int kb = kbeg + st * KS;
            if (kb + KS <= kend) {
#pragma unroll
                for (int j = 0; j < 16; ++j) dst[j] = ld_buf(ra, lane_off, kb * (int)sizeof(T) + 64 * j);
            } else {   // the slice end: chunks past it load from an out-of-range offset (zeros)
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    dst[j] = ld_buf(ra, kb + 32 * j + 8 * grp < kend ? lane_off : 0x80000000u, kb * (int)sizeof(T) + 64 * j);
            }
        };
        // the step's 16 x 512 vector slice: thread t moves chunks t + 256 i (vector c / 64,
        // k chunk c % 64); vectors past N and k past the slice load from an out-of-range
        // offset (zeros)
        auto load_x = [&](int st, uint4 (&dst)[4]) {
            const int kb = kbeg + st * KS;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = tid + 256 * i, n = c >> 6, kc = 8 * (c & 63);
                const uint32_t off = n < g.N && kb + kc < kend ? x_off[i] : 0x80000000u;
                dst[i] = ld_buf(rb, off, kb * (int)sizeof(T));
            }
        };
        auto store_x = [&](int buf, const uint4 (&src)[4]) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = tid + 256 * i;
                *(uint4 *)&xs[buf][c >> 6][8 * (c & 63)] = src[i];
            }
        };
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        // vector fragments are read two MFMAs ahead (not all 16 up front: registers)
        auto compute = [&](const uint4 (&wr)[16], int buf) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint4 xf = *(const uint4 *)&xs[buf][r][32 * j + 8 * grp];
                acc = mma16x16<T>(xf, wr[j], acc);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int j = 0; j < 14; ++j) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        };

        // matrix chunks one step ahead (wa / wb), vector slices two steps ahead (xa / xb), so
        // every wait is for loads issued a whole step earlier
        uint4 wa[16], wb[16], xa[4], xb[4];
        if (nsteps > 0) {
            load_x(0, xa);
            if (nsteps > 1) load_x(1, xb);
            load_w(0, wa);
            store_x(0, xa);
            __syncthreads();
        }
        for (int st = 0; st < nsteps; st += 2) {
            // step st: matrix chunks in wa, vectors in xs[0]
            const bool more1 = st + 1 < nsteps;
            if (more1) load_w(st + 1, wb);
            if (st + 2 < nsteps) load_x(st + 2, xa);
            compute(wa, 0);
            if (more1) store_x(1, xb);
            __syncthreads();   // xs[1] written; every wave is done with xs[0]
            if (!more1) break;
            // step st + 1: matrix chunks in wb, vectors in xs[1]
            const bool more2 = st + 2 < nsteps;
            if (more2) load_w(st + 2, wa);
            if (st + 3 < nsteps) load_x(st + 3, xb);
            compute(wb, 1);
            if (more2) store_x(0, xa);
            __syncthreads();
        }

        const int m = m0 + r;
        if (m < g.M) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = 4 * grp + i;
                if (n >= g.N) continue;
                if (g.splits > 1) {
                    float *ws = (float *)g.ws + ((int64_t)ks * g.batch + bz) * g.M * (int64_t)g.N;
                    ws[(int64_t)m * g.N + n] = acc[i];
                } else {
                    T *c = (T *)g.c + bz * g.c_bs + m * g.c_rs + n * g.c_cs;
                    store_out<T>(g, c, acc[i], bz * g.bias_bs + m * g.bias_rs + n * g.bias_cs);
                }
            }
        }
        __syncthreads();   // xs reuse by the next batch iteration
    }
}

// ---- k_thin_dot4: the K-contiguous matrix read as 4-row x 1 KiB streams --------------------
// A probe that only streams a 16384^2 bf16 matrix reached 0.81 of 8 TB/s when each CU keeps
// ~8 rows in flight, 4 waves reading consecutive 1 KiB pieces of the same rows, each load
// instruction covering 4 rows x 256 bytes; with 16 rows per wave (the 16 x 16 MFMA layout of
// k_thin_dot) it reached 0.58.  v_mfma_f32_4x4x4bf16_1k runs 16 independent 4 x 4 x 4 blocks:
// lane 4 b + i holds row i of block b's A and column i of its B, and receives D_b[0..3][i].
// Here block b is a k chunk, so one 16-byte load per lane (row i, 8 k) covers 4 rows x 128 k,
// the two 4-k halves feed two MFMAs, and the 16 blocks' partial sums are added across lanes
// after each row quad.
//
// Workgroup: 4 waves on the same row quad; wave w takes k quarter w of the workgroup's K
// slice (kq = k_chunk / 4 = 128 U) and keeps that quarter of the vectors in registers for
// every row quad it visits (G groups of 4 vectors).  Row quads rq = blockIdx.x + gridDim.x t;
// the 4 quarters' sums meet in LDS.  The host guarantees k_chunk = 512 U, K % 8 == 0, N <= 4G,
// and 31-bit offsets for the whole matrix and vector block.
typedef __bf16 bf16x4t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4t __attribute__((ext_vector_type(4)));

template <class T> __device__ __forceinline__ f32x4 mma4x4(uint2 a, uint2 b, f32x4 c);
template <> __device__ __forceinline__ f32x4 mma4x4<bf16_t>(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(bf16x4t, a), __builtin_bit_cast(bf16x4t, b), c,
                                                  0, 0, 0);
}
template <> __device__ __forceinline__ f32x4 mma4x4<f16_t>(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4t, a), __builtin_bit_cast(f16x4t, b), c, 0, 0, 0);
}

constexpr int kDot4U = 8;   // 16-byte loads per lane per row quad (k quarter = 1024)
static_assert(kThinDot4Chunk == 512 * kDot4U, "K slice of k_thin_dot4");

template <class T, int G>
__global__ __launch_bounds__(256) void k_thin_dot4(GemmArgs g) {
    constexpr int U = kDot4U;
    __shared__ float red[2][4][G][4][4];   // [parity][wave][group][row][column]
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 3, b = lane >> 2;   // row / column index in the block; block = k chunk
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);
    const int kq0 = kbeg + w * (g.k_chunk >> 2);    // this wave's k quarter
    const bool full = kq0 + 128 * U <= kend;         // no chunk of the quarter is past the slice
    const int nquads = cdiv(g.M, 4);
    const uint4 zero = make_uint4(0, 0, 0, 0);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const __amdgpu_buffer_rsrc_t ra = buf_rsrc((const T *)g.a + bz * g.a_bs);
        const __amdgpu_buffer_rsrc_t rb = buf_rsrc((const T *)g.b + bz * g.b_bs);
        // this lane's vector chunks: vector 4 q + i, k = kq0 + 128 u + 8 b
        uint4 xr[G][U];
#pragma unroll
        for (int q = 0; q < G; ++q)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int n = 4 * q + i, k = kq0 + 128 * u + 8 * b;
                const uint32_t off = n < g.N && k < kend ? (uint32_t)(((int64_t)n * g.b_cs + k) * sizeof(T)) : 0x80000000u;
                xr[q][u] = ld_buf(rb, off, 0);
            }
        // matrix chunks of row quad rq: row 4 rq + i (clamped), k = kq0 + 128 u + 8 b
        auto load_w = [&](int rq, uint4 (&dst)[U]) {
            const int row = min(4 * rq + i, g.M - 1);
            const uint32_t base = (uint32_t)(((int64_t)row * g.a_rs + kq0 + 8 * b) * sizeof(T));
            if (full) {
#pragma unroll
                for (int u = 0; u < U; ++u) dst[u] = ld_buf(ra, base, 256 * u * (int)(sizeof(T) / 2));
            } else {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    dst[u] = ld_buf(ra, kq0 + 128 * u + 8 * b < kend ? base : 0x80000000u, 256 * u * (int)(sizeof(T) / 2));
            }
        };
        auto quad = [&](int rq, const uint4 (&wr)[U], int parity) {
            f32x4 acc[G];
#pragma unroll
            for (int q = 0; q < G; ++q) acc[q] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int q = 0; q < G; ++q) {
                    acc[q] = mma4x4<T>(make_uint2(wr[u].x, wr[u].y), make_uint2(xr[q][u].x, xr[q][u].y), acc[q]);
                    acc[q] = mma4x4<T>(make_uint2(wr[u].z, wr[u].w), make_uint2(xr[q][u].z, xr[q][u].w), acc[q]);
                }
            // sum the 16 k-chunk blocks: lanes i, i + 4, ..., i + 60
#pragma unroll
            for (int q = 0; q < G; ++q)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = acc[q][r];
                    v += __shfl_xor(v, 4, 64);
                    v += __shfl_xor(v, 8, 64);
                    v += __shfl_xor(v, 16, 64);
                    v += __shfl_xor(v, 32, 64);
                    acc[q][r] = v;
                }
            if (lane < 4) {
#pragma unroll
                for (int q = 0; q < G; ++q)
#pragma unroll
                    for (int r = 0; r < 4; ++r) red[parity][w][q][r][i] = acc[q][r];
            }
            __syncthreads();
            // thread t < 16 G: group q = t / 16, row r = (t / 4) % 4, column c = t % 4
            if (tid < 16 * G) {
                const int q = tid >> 4, r = (tid >> 2) & 3, c = tid & 3;
                const float v = red[parity][0][q][r][c] + red[parity][1][q][r][c] + red[parity][2][q][r][c] +
                                red[parity][3][q][r][c];
                const int m = 4 * rq + r, n = 4 * q + c;
                if (m < g.M && n < g.N) {
                    if (g.splits > 1) {
                        float *ws = (float *)g.ws + ((int64_t)ks * g.batch + bz) * g.M * (int64_t)g.N;
                        ws[(int64_t)m * g.N + n] = v;
                    } else {
                        T *cp = (T *)g.c + bz * g.c_bs + m * g.c_rs + n * g.c_cs;
                        store_out<T>(g, cp, v, bz * g.bias_bs + m * g.bias_rs + n * g.bias_cs);
                    }
                }
            }
        };

        // three row quads of matrix chunks in flight (wa, wb, wc rotate)
        uint4 wa[U], wb[U], wc[U];
        const int step = gridDim.x;
        int rq = blockIdx.x;
        if (rq < nquads) load_w(rq, wa);
        if (rq + step < nquads) load_w(rq + step, wb);
        int parity = 0;
        while (rq < nquads) {
            if (rq + 2 * step < nquads) load_w(rq + 2 * step, wc);
            quad(rq, wa, parity);
            parity ^= 1;
            rq += step;
            if (rq >= nquads) break;
            if (rq + 2 * step < nquads) load_w(rq + 2 * step, wa);
            quad(rq, wb, parity);
            parity ^= 1;
            rq += step;
            if (rq >= nquads) break;
            if (rq + 2 * step < nquads) load_w(rq + 2 * step, wb);
            quad(rq, wc, parity);
            parity ^= 1;
            rq += step;
        }
        __syncthreads();   // red reuse by the next batch iteration
    }
}

// ---- k_dotx: up to 8 vectors against a K-contiguous matrix, the whole K in one workgroup ----
// The k_thin_dot4 stream (4 rows x 256 bytes per load instruction, v_mfma_f32_4x4x4 with one
// k chunk per 4-lane block) without K slices: wave w of the NW-wave workgroup owns k
// [1024 w, 1024 w + 1024) and keeps that piece of the 8 vectors in registers (2 groups x 8
// chunks), so no partial planes and no reduction launch are needed.  A workgroup walks a
// group of 16 row quads; after each quad the 16 k-chunk blocks are summed across lanes (DPP
// row rotations, then lanes 16 / 32 apart) and lanes 0..3 park the quad's 4 x 8 sums in LDS;
// after the group the NW waves' sums are added in wave order (deterministic) and stored with
// the epilogue.  The matrix is read with non-temporal loads (it is streamed once).
//
// Vectors: K-contiguous (XKC, vector n at n * b_cs + k), or the natural K x 8 row-major block
// (element (k, n) at k * b_rs + n, 16-byte rows), which each wave transposes through its own
// LDS region in 256-row phases.  Measured on MI355X, 16384^2 bf16 matrix x 8 vectors:
// 82.2-83.3 us natural / 81.9 us K-contiguous (0.81 / 0.82 of 8 TB/s); 92 us with cached
// loads, 84-85 us with workgroup barriers between the transpose phases.
// The host guarantees N <= 8, K % 8 == 0, K <= NW * 1024, batch <= 65535 and 31-bit offsets.
constexpr int kDotxPH = 256;                   // natural vector rows per LDS transpose phase
constexpr int kDotxPitch = 2 * kDotxPH + 64;   // bytes per vector row of a phase (conflict-free reads)

__device__ __forceinline__ uint4 ld_buf_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, int soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);   // nt
    return make_uint4(v[0], v[1], v[2], v[3]);
}
// Orders one wave's LDS accesses across its lanes: the LDS executes a wave's instructions in
// issue order, so only the compiler has to keep them in program order (no workgroup barrier).
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// sum over the 16 lanes l' with l' % 4 == l % 4 (the k-chunk blocks of a 4 x 4 MFMA result)
__device__ __forceinline__ float sum_blocks(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

template <class T, int NW, bool XKC>
__global__ __launch_bounds__(64 * NW) void k_dotx(GemmArgs g) {
    constexpr int U = kDotxU, G = 2, KW = kDotxKW, QG = kDotxQG;
    // the natural vectors' transpose regions (one per wave) and the cross-wave sums apart, so
    // no wave waits for another before its first quad
    constexpr int XB = XKC ? 0 : NW * 8 * kDotxPitch, RB = NW * QG * 32 * 4;
    __shared__ __attribute__((aligned(16))) char lds[XB + RB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 3, b = lane >> 2;   // row / column index in the 4 x 4 block; block = k chunk
    const int kw = w * KW;
    const bool full = kw + KW <= g.K;
    const int nquads = cdiv(g.M, 4);
    const int bz = blockIdx.z;
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc((const T *)g.a + bz * g.a_bs);
    const __amdgpu_buffer_rsrc_t rb = buf_rsrc((const T *)g.b + bz * g.b_bs);
    // the matrix chunks of row quad rq: row 4 rq + i (clamped), k = kw + 128 u + 8 b
    auto load_w = [&](int rq, uint4 (&dst)[U]) {
        const int row = min(4 * rq + i, g.M - 1);
        const uint32_t base = (uint32_t)(((int64_t)row * g.a_rs + kw + 8 * b) * sizeof(T));
        if (full) {
#pragma unroll
            for (int u = 0; u < U; ++u) dst[u] = ld_buf_nt(ra, base, 256 * u);
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) dst[u] = ld_buf_nt(ra, kw + 128 * u + 8 * b < g.K ? base : kOOB, 256 * u);
        }
    };
    int grp = blockIdx.x;
    uint4 wa[U];
    if (grp * QG < nquads) load_w(grp * QG, wa);   // in flight while the vectors are loaded
    // this lane's vector chunks: vector 4 q + i, k = kw + 128 u + 8 b
    uint4 xr[G][U];
    if constexpr (XKC) {
#pragma unroll
        for (int q = 0; q < G; ++q)
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int n = 4 * q + i, k = kw + 128 * u + 8 * b;
                const uint32_t off = n < g.N && k < g.K ? (uint32_t)(((int64_t)n * g.b_cs + k) * sizeof(T)) : kOOB;
                xr[q][u] = ld_buf(rb, off, 0);
            }
    } else {
        // natural rows: lane l takes row pairs (2 l, 2 l + 1) and (2 l + 128, 2 l + 129) of a
        // phase, packs each vector's two values into one dword and stores it at [n][k]; the
        // next phase's rows are in flight meanwhile
        char *my = lds + w * 8 * kDotxPitch;
        constexpr int NPH = KW / kDotxPH;
        uint4 r0[2][2], r1[2][2];
        auto xload = [&](int ph, uint4 (&d0)[2], uint4 (&d1)[2]) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int k = kw + kDotxPH * ph + 2 * (lane + 64 * j);   // even: k + 1 < K iff k < K
                const bool in = k < g.K;
                d0[j] = ld_buf(rb, in ? (uint32_t)((int64_t)k * g.b_rs * sizeof(T)) : kOOB, 0);
                d1[j] = ld_buf(rb, in ? (uint32_t)((int64_t)(k + 1) * g.b_rs * sizeof(T)) : kOOB, 0);
            }
        };
        xload(0, r0[0], r1[0]);
        xload(1, r0[1], r1[1]);
#pragma unroll
        for (int ph = 0; ph < NPH; ++ph) {
            const int s = ph & 1;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t a0[4] = {r0[s][j].x, r0[s][j].y, r0[s][j].z, r0[s][j].w};
                const uint32_t a1[4] = {r1[s][j].x, r1[s][j].y, r1[s][j].z, r1[s][j].w};
#pragma unroll
                for (int n = 0; n < 8; ++n) {
                    const uint32_t lo = a0[n >> 1], hi = a1[n >> 1];
                    const uint32_t v = (n & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                    *(uint32_t *)(my + n * kDotxPitch + 4 * (lane + 64 * j)) = v;
                }
            }
            if (ph + 2 < NPH) xload(ph + 2, r0[s], r1[s]);
            wave_lds_order();   // the region is the wave's own: its lanes' writes before the reads
#pragma unroll
            for (int up = 0; up < 2; ++up)
#pragma unroll
                for (int q = 0; q < G; ++q)
                    xr[q][2 * ph + up] = *(const uint4 *)(my + (4 * q + i) * kDotxPitch + 256 * up + 16 * b);
            wave_lds_order();   // the reads before the next phase's writes
        }
    }
    float *red = (float *)(lds + XB);   // [wave][quad of the group][group q][column i][row r]
    for (; grp * QG < nquads; grp += gridDim.x) {
        const int q0 = grp * QG;
        for (int t = 0; t < QG; ++t) {
            f32x4 acc[G];
#pragma unroll
            for (int q = 0; q < G; ++q) acc[q] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int q = 0; q < G; ++q) {
                    acc[q] = mma4x4<T>(make_uint2(wa[u].x, wa[u].y), make_uint2(xr[q][u].x, xr[q][u].y), acc[q]);
                    acc[q] = mma4x4<T>(make_uint2(wa[u].z, wa[u].w), make_uint2(xr[q][u].z, xr[q][u].w), acc[q]);
                }
            // the next quad's loads reuse wa: kept after the MFMAs (one buffer per wave; the
            // workgroup's NW waves keep the loads in flight)
            __builtin_amdgcn_sched_barrier(0);
            const int nrq = t + 1 < QG ? q0 + t + 1 : (grp + gridDim.x) * QG;
            if (nrq < nquads) load_w(nrq, wa);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < G; ++q) {
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[q][r] = sum_blocks(acc[q][r]);
                if (lane < 4) *(f32x4 *)&red[w * QG * 32 + t * 32 + q * 16 + i * 4] = acc[q];
            }
        }
        __syncthreads();
        for (int o = tid; o < QG * 32; o += 64 * NW) {
            float v = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) v += red[ww * QG * 32 + o];
            const int t = o >> 5, q = (o >> 4) & 1, c = (o >> 2) & 3, r = o & 3;
            const int row = 4 * (q0 + t) + r, n = 4 * q + c;
            if (row < g.M && n < g.N) {
                T *cp = (T *)g.c + bz * g.c_bs + (int64_t)row * g.c_rs + n * g.c_cs;
                store_out<T>(g, cp, v, bz * g.bias_bs + (int64_t)row * g.bias_rs + n * g.bias_cs);
            }
        }
        __syncthreads();   // red is rewritten by the next group
    }
}

template <class T, bool XKC>
hipError_t launch_dotx_t(int nw, const GemmArgs &g, dim3 grid, hipStream_t st) {
    switch (nw) {
    case 1: hipLaunchKernelGGL((k_dotx<T, 1, XKC>), grid, dim3(64), 0, st, g); break;
    case 2: hipLaunchKernelGGL((k_dotx<T, 2, XKC>), grid, dim3(128), 0, st, g); break;
    case 4: hipLaunchKernelGGL((k_dotx<T, 4, XKC>), grid, dim3(256), 0, st, g); break;
    case 8: hipLaunchKernelGGL((k_dotx<T, 8, XKC>), grid, dim3(512), 0, st, g); break;
    case 16: hipLaunchKernelGGL((k_dotx<T, 16, XKC>), grid, dim3(1024), 0, st, g); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

int dotx_waves(int64_t K) {
    const int64_t need = (K + kDotxKW - 1) / kDotxKW;
    int nw = 1;
    while (nw < need) nw *= 2;
    return nw;
}

bool dotx_offsets_fit(const GemmArgs &g, bool xkc) {
    const int64_t lim = (int64_t)1 << 31;
    const int64_t xb = xkc ? (int64_t)8 * g.b_cs + g.K : ((int64_t)g.K + 1) * g.b_rs;
    return ((int64_t)g.M * g.a_rs + g.K) * 2 < lim && xb * 2 < lim;
}

// k_thin_dot addresses 16 rows of A (16 vectors of B) plus a K slice from one buffer
// resource: 31-bit offsets
bool thin_dot_offsets_fit(const GemmArgs &g) {
    const int64_t lim = (int64_t)1 << 31;
    return (16 * g.a_rs + g.K + 512) * 2 < lim && (16 * g.b_cs + g.K + 512) * 2 < lim;
}

bool thin_dot4_offsets_fit(const GemmArgs &g) {
    const int64_t lim = (int64_t)1 << 31;
    return ((int64_t)g.M * g.a_rs + g.K) * 2 < lim && ((int64_t)16 * g.b_cs + g.K) * 2 < lim;
}

hipError_t launch_thin(int dt, bool ktail, const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid,
                       hipStream_t st) {
    if (t.bm == 4 && t.bn == 8) {   // k_dotx: grid (row-quad groups, 1, batch)
        // natural vectors: 8 per 16-byte-aligned row; K-contiguous: 16-byte-aligned vector rows
        const bool ok_b = b_kc ? (g.b_cs & 7) == 0 && ((uintptr_t)g.b & 15) == 0
                               : g.N == 8 && g.b_cs == 1 && (g.b_rs & 7) == 0 && ((uintptr_t)g.b & 15) == 0;
        if (!a_kc || !ok_b || g.N > 8 || (g.K & 7) || g.K > (int64_t)kDotxMaxWaves * kDotxKW || g.splits != 1 ||
            g.persist < 1 || g.batch > 65535 || !dotx_offsets_fit(g, b_kc))
            return hipErrorInvalidValue;
        const dim3 grid2(g.persist, 1, g.batch);
        const int nw = dotx_waves(g.K);
        if (dt == BF16) return b_kc ? launch_dotx_t<bf16_t, true>(nw, g, grid2, st) : launch_dotx_t<bf16_t, false>(nw, g, grid2, st);
        if (dt == F16) return b_kc ? launch_dotx_t<f16_t, true>(nw, g, grid2, st) : launch_dotx_t<f16_t, false>(nw, g, grid2, st);
        return hipErrorInvalidValue;
    }
    if (t.bm == 4 && t.bn == 16) {   // k_thin_dot4: grid (row-quad workgroups, K slices, batch)
        if (!a_kc || !b_kc || g.N > 16 || (g.K & 7) || g.k_chunk != 512 * kDot4U || g.persist < 1 ||
            !thin_dot4_offsets_fit(g))
            return hipErrorInvalidValue;
        dim3 grid2(g.persist, g.splits, grid.z);
        const int G = (g.N + 3) / 4;
#define MB_DOT4(GG) hipLaunchKernelGGL((k_thin_dot4<TT, GG>), grid2, dim3(256), 0, st, g)
        if (dt == BF16) {
            using TT = bf16_t;
            if (G == 1) MB_DOT4(1); else if (G == 2) MB_DOT4(2); else if (G == 3) MB_DOT4(3); else MB_DOT4(4);
        } else if (dt == F16) {
            using TT = f16_t;
            if (G == 1) MB_DOT4(1); else if (G == 2) MB_DOT4(2); else if (G == 3) MB_DOT4(3); else MB_DOT4(4);
        } else {
            return hipErrorInvalidValue;
        }
#undef MB_DOT4
        return hipGetLastError();
    }
    if (t.bm == 64 && t.bn == 16) {
        if (!a_kc || !b_kc || g.N > 16 || (g.K & 7) || (g.k_chunk & 511) || !thin_dot_offsets_fit(g))
            return hipErrorInvalidValue;
        dim3 grid2(cdiv(g.M, 64), g.splits, grid.z);
        if (dt == BF16) hipLaunchKernelGGL((k_thin_dot<bf16_t>), grid2, dim3(256), 0, st, g);
        else if (dt == F16) hipLaunchKernelGGL((k_thin_dot<f16_t>), grid2, dim3(256), 0, st, g);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    if (dt == BF16)
        return ktail ? launch_thin16<bf16_t, true>(t, a_kc, b_kc, g, grid, st)
                     : launch_thin16<bf16_t, false>(t, a_kc, b_kc, g, grid, st);
    if (dt == F16)
        return ktail ? launch_thin16<f16_t, true>(t, a_kc, b_kc, g, grid, st)
                     : launch_thin16<f16_t, false>(t, a_kc, b_kc, g, grid, st);
    return hipErrorInvalidValue;
}

}  // namespace m16
}  // namespace mb
