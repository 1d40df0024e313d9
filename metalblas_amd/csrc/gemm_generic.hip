// Generic LDS-tiled GEMM for every dtype and any element strides, plus the K==0 fill and
// the split-K reduction.
//
// This is the register-tiled VALU family: it serves int16/int32/int64 (which have no
// matrix-core instruction), and any operand the matrix-core loaders cannot stream
// (unaligned bases, odd leading dimensions, non-unit strides on both axes).  It restates
// the structure of shaders/int_gemm.h:41-154 (A and B staged through shared memory, a
// TM x TN micro-tile per thread, accumulate in ACC_T, truncating store) for wave64:
// BT x BT output tile (BT = 64, 32 or 16), 256 threads as 16x16, (BT/16)^2 accumulators per
// thread, BK = 16 (64, 128 for the smaller tiles).  The small tiles serve products whose
// 64 x 64 tiles would leave CUs idle.
#include "launch.hpp"

#include <type_traits>

namespace mb {

namespace {

template <class T, int BT>
__global__ __launch_bounds__(256) void k_gemm_generic(GemmArgs g) {
    static_assert(BT == 16 || BT == 32 || BT == 64, "generic tile");
    constexpr int GBM = BT, GBN = BT, TT = BT / 16;   // TT x TT outputs per thread
    // K per LDS step: each step is a serial load -> barrier -> compute round, so the small
    // tiles (short per-step compute) take deeper steps, 8 loads per thread per operand
    constexpr int GBK = BT == 16 ? 128 : BT == 32 ? 64 : 16;
    using A = typename Tr<T>::acc;
    __shared__ A As[GBK][GBM + 1];
    __shared__ A Bs[GBK][GBN + 1];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int tiles_n = cdiv(g.N, GBN);
    const int m0 = (blockIdx.x / tiles_n) * GBM;
    const int n0 = (blockIdx.x % tiles_n) * GBN;
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);
    const bool a_kc = g.a_cs == 1;   // A row-major: consecutive threads walk K
    const bool b_kc = g.b_rs == 1;   // B column-major: consecutive threads walk K

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const T *Ab = (const T *)g.a + bz * g.a_bs;
        const T *Bb = (const T *)g.b + bz * g.b_bs;
        A acc[TT][TT];
#pragma unroll
        for (int i = 0; i < TT; ++i)
#pragma unroll
            for (int j = 0; j < TT; ++j) acc[i][j] = Tr<T>::zero();

        for (int k0 = kbeg; k0 < kend; k0 += GBK) {
#pragma unroll
            for (int i = 0; i < (GBM * GBK) / 256; ++i) {
                const int idx = tid + 256 * i;
                const int m = a_kc ? idx / GBK : idx % GBM;
                const int k = a_kc ? idx % GBK : idx / GBM;
                const int gm = m0 + m, gk = k0 + k;
                A v = Tr<T>::zero();
                if (gm < g.M && gk < kend) v = Tr<T>::up(Ab[gm * g.a_rs + gk * g.a_cs], g.conj_a);
                As[k][m] = v;
            }
#pragma unroll
            for (int i = 0; i < (GBN * GBK) / 256; ++i) {
                const int idx = tid + 256 * i;
                const int n = b_kc ? idx / GBK : idx % GBN;
                const int k = b_kc ? idx % GBK : idx / GBN;
                const int gn = n0 + n, gk = k0 + k;
                A v = Tr<T>::zero();
                if (gn < g.N && gk < kend) v = Tr<T>::up(Bb[gk * g.b_rs + gn * g.b_cs], g.conj_b);
                Bs[k][n] = v;
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < GBK; ++kk) {
                A av[TT], bv[TT];
#pragma unroll
                for (int i = 0; i < TT; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
                for (int j = 0; j < TT; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
                for (int i = 0; i < TT; ++i)
#pragma unroll
                    for (int j = 0; j < TT; ++j) acc[i][j] = Tr<T>::mac(acc[i][j], av[i], bv[j]);
            }
            __syncthreads();
        }

        T *Cb = (T *)g.c + bz * g.c_bs;
#pragma unroll
        for (int i = 0; i < TT; ++i) {
            const int gm = m0 + ty + 16 * i;
            if (gm >= g.M) continue;
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                const int gn = n0 + tx + 16 * j;
                if (gn >= g.N) continue;
                if (g.splits > 1) {
                    A *ws = (A *)g.ws;
                    ws[(((int64_t)ks * g.batch + bz) * g.M + gm) * g.N + gn] = acc[i][j];
                } else {
                    store_out<T>(g, Cb + gm * g.c_rs + gn * g.c_cs, acc[i][j],
                                 bz * g.bias_bs + gm * g.bias_rs + gn * g.bias_cs);
                }
            }
        }
    }
}

// K == 0: C = beta*bias (epilogue with a zero product) or 0.
template <class T>
__global__ __launch_bounds__(256) void k_fill(GemmArgs g) {
    const int64_t total = (int64_t)g.batch * g.M * g.N;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t bz = i / ((int64_t)g.M * g.N);
        const int64_t r = i % ((int64_t)g.M * g.N);
        const int64_t m = r / g.N, n = r % g.N;
        T *c = (T *)g.c + bz * g.c_bs + m * g.c_rs + n * g.c_cs;
        store_out<T>(g, c, Tr<T>::zero(), bz * g.bias_bs + m * g.bias_rs + n * g.bias_cs);
    }
}

// Split-K: C = epilogue(sum_s ws[s]).  TPO threads share one output: thread `sub` sums
// planes sub, sub+TPO, ... (four independent partial sums), and the TPO partials are added
// in a fixed order through LDS, so the result is deterministic.  Threads with the same sub
// read consecutive outputs (coalesced).
template <class T, int TPO>
__global__ __launch_bounds__(256) void k_splitk_reduce(GemmArgs g) {
    using A = typename Tr<T>::acc;
    constexpr int OPB = 256 / TPO;   // outputs per block iteration
    __shared__ A part[TPO][OPB];
    const int64_t plane = (int64_t)g.batch * g.M * g.N;
    const A *ws = (const A *)g.ws;
    const int sub = threadIdx.x / OPB, oi = threadIdx.x % OPB;
    for (int64_t base = (int64_t)blockIdx.x * OPB; base < plane; base += (int64_t)gridDim.x * OPB) {
        const int64_t i = base + oi;
        A v0 = Tr<T>::zero(), v1 = v0, v2 = v0, v3 = v0;
        if (i < plane) {
            int s = sub;
            for (; s + 3 * TPO < g.splits; s += 4 * TPO) {
                v0 = acc_add(v0, ws[(int64_t)s * plane + i]);
                v1 = acc_add(v1, ws[(int64_t)(s + TPO) * plane + i]);
                v2 = acc_add(v2, ws[(int64_t)(s + 2 * TPO) * plane + i]);
                v3 = acc_add(v3, ws[(int64_t)(s + 3 * TPO) * plane + i]);
            }
            for (; s < g.splits; s += TPO) v0 = acc_add(v0, ws[(int64_t)s * plane + i]);
        }
        part[sub][oi] = acc_add(acc_add(v0, v1), acc_add(v2, v3));
        __syncthreads();
        if (sub == 0 && i < plane) {
            A v = part[0][oi];
#pragma unroll
            for (int q = 1; q < TPO; ++q) v = acc_add(v, part[q][oi]);
            const int64_t bz = i / ((int64_t)g.M * g.N);
            const int64_t r = i % ((int64_t)g.M * g.N);
            const int64_t m = r / g.N, n = r % g.N;
            T *c = (T *)g.c + bz * g.c_bs + m * g.c_rs + n * g.c_cs;
            store_out<T>(g, c, v, bz * g.bias_bs + m * g.bias_rs + n * g.bias_cs);
        }
        __syncthreads();
    }
}

// The same reduction for fp32 partials with N % 4 == 0: each thread sums 4 consecutive outputs
// of one row with 16-byte loads (same summation order per output as k_splitk_reduce).
template <class T, int TPO>
__global__ __launch_bounds__(256) void k_splitk_reduce4(GemmArgs g) {
    constexpr int OPB = 256 / TPO;   // 4-output groups per block iteration
    __shared__ float4 part[TPO][OPB];
    const int64_t plane = (int64_t)g.batch * g.M * g.N;
    const int64_t groups = plane / 4;
    const float4 *ws = (const float4 *)g.ws;
    const int sub = threadIdx.x / OPB, oi = threadIdx.x % OPB;
    auto add = [](float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); };
    for (int64_t base = (int64_t)blockIdx.x * OPB; base < groups; base += (int64_t)gridDim.x * OPB) {
        const int64_t i = base + oi;
        float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0, v2 = v0, v3 = v0;
        if (i < groups) {
            int s = sub;
            for (; s + 3 * TPO < g.splits; s += 4 * TPO) {
                v0 = add(v0, ws[(int64_t)s * groups + i]);
                v1 = add(v1, ws[(int64_t)(s + TPO) * groups + i]);
                v2 = add(v2, ws[(int64_t)(s + 2 * TPO) * groups + i]);
                v3 = add(v3, ws[(int64_t)(s + 3 * TPO) * groups + i]);
            }
            for (; s < g.splits; s += TPO) v0 = add(v0, ws[(int64_t)s * groups + i]);
        }
        part[sub][oi] = add(add(v0, v1), add(v2, v3));
        __syncthreads();
        if (sub == 0 && i < groups) {
            float4 v = part[0][oi];
#pragma unroll
            for (int q = 1; q < TPO; ++q) v = add(v, part[q][oi]);
            const int64_t e = 4 * i;
            const int64_t bz = e / ((int64_t)g.M * g.N);
            const int64_t r = e % ((int64_t)g.M * g.N);
            const int64_t m = r / g.N, n = r % g.N;   // n % 4 == 0: the 4 outputs share row m
            T *c = (T *)g.c + bz * g.c_bs + m * g.c_rs;
            const int64_t bo = bz * g.bias_bs + m * g.bias_rs;
            const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) store_out<T>(g, c + (n + q) * g.c_cs, vv[q], bo + (n + q) * g.bias_cs);
        }
        __syncthreads();
    }
}

// Operand copy (PackArgs): each thread writes 4 consecutive elements along the destination's
// contiguous dimension (coalesced stores); source reads follow the source strides.  The grid
// is x: inner chunks, y: outer index (grid-stride), z: batch (grid-stride).
template <class E>
__global__ __launch_bounds__(256) void k_pack(PackArgs a) {
    const int64_t inner_n = a.contig_cols ? a.cols_p : a.rows_p;
    const int64_t outer_n = a.contig_cols ? a.rows_p : a.cols_p;
    const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 >= inner_n) return;
    for (int64_t bz = blockIdx.z; bz < a.batch; bz += gridDim.z) {
        const E *src = (const E *)a.src + bz * a.s_bs;
        E *dst = (E *)a.dst + bz * a.d_bs;
        for (int64_t o = blockIdx.y; o < outer_n; o += gridDim.y) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t i = i0 + j;
                if (i >= inner_n) break;
                const int64_t r = a.contig_cols ? o : i, c = a.contig_cols ? i : o;
                E v = E(0);
                if (r < a.rows && c < a.cols) v = src[r * a.s_rs + c * a.s_cs];
                dst[r * a.d_rs + c * a.d_cs] = v;
            }
        }
    }
}

// 16-bit rows whose source is contiguous along the row but at any 2-byte alignment (storage
// offsets such as the reference's 17-element offset, odd leading dimensions), copied into
// 16-byte aligned, zero-padded destination rows: each thread writes 8 elements with one
// 16-byte store, cut out of the two aligned 16-byte source chunks that cover them (whole-chunk
// loads: a load instruction reads 1 KiB of consecutive row bytes).  Every thread of a row
// shares the row's misalignment (8-element chunks are 16 bytes), so the cut is wave-uniform.
// The second chunk is read only when it starts before the row's end, so every read lies in a
// page that holds a valid element.  Grid as k_pack, with 8-element chunks.
__device__ __forceinline__ void pack16_rows(const PackArgs &a, int64_t ci) {
    const int64_t chunks = a.cols_p / 8;
    if (ci >= chunks) return;
    const int64_t c0 = ci * 8;
    for (int64_t bz = blockIdx.z; bz < a.batch; bz += gridDim.z) {
        const uint16_t *src = (const uint16_t *)a.src + bz * a.s_bs;
        uint16_t *dst = (uint16_t *)a.dst + bz * a.d_bs;
        for (int64_t r = blockIdx.y; r < a.rows_p; r += gridDim.y) {
            uint32_t o[4] = {0u, 0u, 0u, 0u};
            if (r < a.rows && c0 < a.cols) {
                const uint16_t *row = src + r * a.s_rs;
                const int mis = (int)((uintptr_t)(row + c0) & 15);   // 0, 2, ..., 14; row-uniform
                const uint4 *w = (const uint4 *)((const char *)(row + c0) - mis);
                const int64_t left = (a.cols - c0) * 2 + mis;   // bytes from w[0] to the row end
                const uint4 lo = w[0];
                const uint4 hi = left > 16 ? w[1] : make_uint4(0u, 0u, 0u, 0u);
                const uint32_t d[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                const int q = mis >> 2, sh = mis & 3;
                // the 5 words from word q on, picked with uniform selects
                uint32_t e[5];
#pragma unroll
                for (int j = 0; j < 5; ++j)
                    e[j] = q == 0 ? d[j] : q == 1 ? d[j + 1] : q == 2 ? d[j + 2] : d[j + 3];
#pragma unroll
                for (int k = 0; k < 4; ++k) o[k] = __builtin_amdgcn_alignbyte(e[k + 1], e[k], sh);
                const int64_t valid = a.cols - c0;   // elements of this chunk inside the row
                if (valid < 8) {
#pragma unroll
                    for (int x = 0; x < 8; ++x)
                        if (x >= valid) o[x >> 1] &= (x & 1) ? 0x0000ffffu : 0xffff0000u;
                }
            }
            uint4 v;
            v.x = o[0];
            v.y = o[1];
            v.z = o[2];
            v.w = o[3];
            *(uint4 *)(dst + r * a.d_rs + c0) = v;
        }
    }
}

__global__ __launch_bounds__(256) void k_pack16_rows(PackArgs a) {
    pack16_rows(a, (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// Both operands of a product in one launch: blocks [0, nx0) of x copy a0, the rest a1 (rows
// and batches grid-stride over the shared y and z extents).  One launch instead of two saves
// the second dispatch and its ramp-up (both operands are copied for misaligned rows).
__global__ __launch_bounds__(256) void k_pack16_rows2(PackArgs a0, PackArgs a1, int nx0) {
    if ((int)blockIdx.x < nx0)
        pack16_rows(a0, (int64_t)blockIdx.x * 256 + threadIdx.x);
    else
        pack16_rows(a1, (int64_t)(blockIdx.x - nx0) * 256 + threadIdx.x);
}

// Bhat expansion (CplxExpandArgs): thread per (n, k pair-block) writes the two K-adjacent
// pairs of Bhat's columns 2n and 2n + 1; the padding k' in [2K, ld) is zero-filled.
template <class R>
__global__ __launch_bounds__(256) void k_cplx_expand(CplxExpandArgs a) {
    const int64_t kp = a.ld / 2;   // complex k positions per Bhat column, padding included
    const int64_t total = (int64_t)a.N * kp;
    const R sa = a.neg_a ? R(-1.f) : R(1.f), sb = a.neg_b ? R(-1.f) : R(1.f);
    for (int64_t bz = blockIdx.y; bz < a.batch; bz += gridDim.y) {
        const R *src = (const R *)a.b + 2 * bz * a.b_bs;
        R *dst = (R *)a.dst + bz * a.d_bs;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
            const int64_t n = i / kp, k = i % kp;
            R re = R(0.f), im = R(0.f);
            if (k < a.K) {
                const R *e = src + 2 * (k * a.b_rs + n * a.b_cs);
                re = e[0];
                im = e[1];
            }
            R *c0 = dst + (2 * n) * a.ld + 2 * k;        // column 2n: (re, -sa sb im)
            R *c1 = dst + (2 * n + 1) * a.ld + 2 * k;    // column 2n+1: (sb im, sa re)
            c0[0] = re;
            c0[1] = -(sa * sb) * im;
            c1[0] = sb * im;
            c1[1] = sa * re;
        }
    }
}

inline int elementwise_blocks(int64_t total) {
    int64_t b = (total + 255) / 256;
    return (int)(b < 65536 ? (b < 1 ? 1 : b) : 65536);
}

}  // namespace

hipError_t launch_cplx_expand(const CplxExpandArgs &a, hipStream_t st) {
    const int64_t total = (int64_t)a.N * (a.ld / 2);
    int64_t blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    dim3 grid((unsigned)(blocks < 1 ? 1 : blocks), (unsigned)(a.batch < 65535 ? a.batch : 65535));
    if (a.half)
        hipLaunchKernelGGL(k_cplx_expand<f16_t>, grid, dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(k_cplx_expand<float>, grid, dim3(256), 0, st, a);
    return hipGetLastError();
}

// 16-bit rows contiguous in source and destination, destination rows 16-byte aligned
static bool pack16_rows_ok(const PackArgs &a) {
    return a.es == 2 && a.contig_cols && a.s_cs == 1 && a.d_cs == 1 && a.cols_p % 8 == 0 && a.d_rs % 8 == 0 &&
           ((uintptr_t)a.dst & 15) == 0 && (a.d_bs % 8) == 0;
}

hipError_t launch_pack2(const PackArgs &a0, const PackArgs &a1, hipStream_t st) {
    if (!pack16_rows_ok(a0) || !pack16_rows_ok(a1)) {
        hipError_t e = launch_pack(a0, st);
        return e != hipSuccess ? e : launch_pack(a1, st);
    }
    const int64_t nx0 = (a0.cols_p / 8 + 255) / 256, nx1 = (a1.cols_p / 8 + 255) / 256;
    const int64_t rows = std::max(a0.rows_p, a1.rows_p), batch = std::max(a0.batch, a1.batch);
    dim3 grid((unsigned)(nx0 + nx1), (unsigned)(rows < 65535 ? rows : 65535), (unsigned)(batch < 65535 ? batch : 65535));
    hipLaunchKernelGGL(k_pack16_rows2, grid, dim3(256), 0, st, a0, a1, (int)nx0);
    return hipGetLastError();
}

hipError_t launch_pack(const PackArgs &a, hipStream_t st) {
    const int64_t inner_n = a.contig_cols ? a.cols_p : a.rows_p;
    const int64_t outer_n = a.contig_cols ? a.rows_p : a.cols_p;
    if (pack16_rows_ok(a)) {
        dim3 grid((unsigned)((a.cols_p / 8 + 255) / 256), (unsigned)(outer_n < 65535 ? outer_n : 65535),
                  (unsigned)(a.batch < 65535 ? a.batch : 65535));
        hipLaunchKernelGGL(k_pack16_rows, grid, dim3(256), 0, st, a);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((inner_n + 1023) / 1024), (unsigned)(outer_n < 65535 ? outer_n : 65535),
              (unsigned)(a.batch < 65535 ? a.batch : 65535));
    switch (a.es) {
        case 1: hipLaunchKernelGGL(k_pack<uint8_t>, grid, dim3(256), 0, st, a); break;
        case 2: hipLaunchKernelGGL(k_pack<uint16_t>, grid, dim3(256), 0, st, a); break;
        case 4: hipLaunchKernelGGL(k_pack<uint32_t>, grid, dim3(256), 0, st, a); break;
        case 8: hipLaunchKernelGGL(k_pack<uint64_t>, grid, dim3(256), 0, st, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_generic(int dt, int bt, const GemmArgs &g, hipStream_t st, LaunchShape *shape) {
    if (bt != 16 && bt != 32 && bt != 64) return hipErrorInvalidValue;
    const int tiles = cdiv(g.M, bt) * cdiv(g.N, bt);
    dim3 grid(tiles, g.splits, g.batch < 65535 ? g.batch : 65535), block(256);
    if (shape) *shape = {grid, block};
    return with_dtype(dt, [&]<class T>() {
        if (bt == 16) hipLaunchKernelGGL((k_gemm_generic<T, 16>), grid, block, 0, st, g);
        else if (bt == 32) hipLaunchKernelGGL((k_gemm_generic<T, 32>), grid, block, 0, st, g);
        else hipLaunchKernelGGL((k_gemm_generic<T, 64>), grid, block, 0, st, g);
        return hipGetLastError();
    });
}

hipError_t launch_fill(int dt, const GemmArgs &g, hipStream_t st) {
    const int blocks = elementwise_blocks((int64_t)g.batch * g.M * g.N);
    return with_dtype(dt, [&]<class T>() {
        hipLaunchKernelGGL(k_fill<T>, dim3(blocks), dim3(256), 0, st, g);
        return hipGetLastError();
    });
}

hipError_t launch_splitk_reduce(int dt, const GemmArgs &g, hipStream_t st) {
    const int64_t plane = (int64_t)g.batch * g.M * g.N;
    // threads per output: enough that a block covers ~8 planes per thread
    const int tpo = g.splits >= 128 ? 16 : g.splits >= 64 ? 8 : (g.splits >= 16 ? 4 : (g.splits >= 4 ? 2 : 1));
    const int64_t opb = 256 / tpo;
    int64_t blocks = (plane + opb - 1) / opb;
    if (blocks > 8192) blocks = 8192;
    return with_dtype(dt, [&]<class T>() {
        if constexpr (std::is_same_v<typename Tr<T>::acc, float>) {
            if (g.N % 4 == 0 && ((uintptr_t)g.ws & 15) == 0) {
                int64_t b4 = (plane / 4 + opb - 1) / opb;
                if (b4 > 8192) b4 = 8192;
                switch (tpo) {
                    case 16: hipLaunchKernelGGL((k_splitk_reduce4<T, 16>), dim3(b4), dim3(256), 0, st, g); break;
                    case 8: hipLaunchKernelGGL((k_splitk_reduce4<T, 8>), dim3(b4), dim3(256), 0, st, g); break;
                    case 4: hipLaunchKernelGGL((k_splitk_reduce4<T, 4>), dim3(b4), dim3(256), 0, st, g); break;
                    case 2: hipLaunchKernelGGL((k_splitk_reduce4<T, 2>), dim3(b4), dim3(256), 0, st, g); break;
                    default: hipLaunchKernelGGL((k_splitk_reduce4<T, 1>), dim3(b4), dim3(256), 0, st, g); break;
                }
                return hipGetLastError();
            }
        }
        switch (tpo) {
            case 16: hipLaunchKernelGGL((k_splitk_reduce<T, 16>), dim3(blocks), dim3(256), 0, st, g); break;
            case 8: hipLaunchKernelGGL((k_splitk_reduce<T, 8>), dim3(blocks), dim3(256), 0, st, g); break;
            case 4: hipLaunchKernelGGL((k_splitk_reduce<T, 4>), dim3(blocks), dim3(256), 0, st, g); break;
            case 2: hipLaunchKernelGGL((k_splitk_reduce<T, 2>), dim3(blocks), dim3(256), 0, st, g); break;
            default: hipLaunchKernelGGL((k_splitk_reduce<T, 1>), dim3(blocks), dim3(256), 0, st, g); break;
        }
        return hipGetLastError();
    });
}

}  // namespace mb
