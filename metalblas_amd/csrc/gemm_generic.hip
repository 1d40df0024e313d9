// Generic LDS-tiled GEMM for every dtype and any element strides, plus the K==0 fill and
// the split-K reduction.
//
// This is the register-tiled VALU family: it serves int16/int32/int64 (which have no
// matrix-core instruction), and any operand the matrix-core loaders cannot stream
// (unaligned bases, odd leading dimensions, non-unit strides on both axes).  It restates
// the structure of shaders/int_gemm.h:41-154 (A and B staged through shared memory, a
// TM x TN micro-tile per thread, accumulate in ACC_T, truncating store) for wave64:
// 64x64 output tile, 256 threads as 16x16, 4x4 accumulators per thread, BK = 16.
#include "launch.hpp"

namespace mb {

namespace {

constexpr int GBM = 64, GBN = 64, GBK = 16;

template <class T>
__global__ __launch_bounds__(256) void k_gemm_generic(GemmArgs g) {
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
        A acc[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = Tr<T>::zero();

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
                A av[4], bv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
                for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[i][j] = Tr<T>::mac(acc[i][j], av[i], bv[j]);
            }
            __syncthreads();
        }

        T *Cb = (T *)g.c + bz * g.c_bs;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int gm = m0 + ty + 16 * i;
            if (gm >= g.M) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
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

// Split-K: C = epilogue(sum_s ws[s]) with a fixed summation order (deterministic).
template <class T>
__global__ __launch_bounds__(256) void k_splitk_reduce(GemmArgs g) {
    using A = typename Tr<T>::acc;
    const int64_t plane = (int64_t)g.batch * g.M * g.N;
    const A *ws = (const A *)g.ws;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < plane; i += (int64_t)gridDim.x * 256) {
        A v = ws[i];
        for (int s = 1; s < g.splits; ++s) v = acc_add(v, ws[s * plane + i]);
        const int64_t bz = i / ((int64_t)g.M * g.N);
        const int64_t r = i % ((int64_t)g.M * g.N);
        const int64_t m = r / g.N, n = r % g.N;
        T *c = (T *)g.c + bz * g.c_bs + m * g.c_rs + n * g.c_cs;
        store_out<T>(g, c, v, bz * g.bias_bs + m * g.bias_rs + n * g.bias_cs);
    }
}

inline int elementwise_blocks(int64_t total) {
    int64_t b = (total + 255) / 256;
    return (int)(b < 65536 ? (b < 1 ? 1 : b) : 65536);
}

}  // namespace

hipError_t launch_generic(int dt, const GemmArgs &g, hipStream_t st, LaunchShape *shape) {
    const int tiles = cdiv(g.M, GBM) * cdiv(g.N, GBN);
    dim3 grid(tiles, g.splits, g.batch < 65535 ? g.batch : 65535), block(256);
    if (shape) *shape = {grid, block};
    return with_dtype(dt, [&]<class T>() {
        hipLaunchKernelGGL(k_gemm_generic<T>, grid, block, 0, st, g);
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
    const int blocks = elementwise_blocks((int64_t)g.batch * g.M * g.N);
    return with_dtype(dt, [&]<class T>() {
        hipLaunchKernelGGL(k_splitk_reduce<T>, dim3(blocks), dim3(256), 0, st, g);
        return hipGetLastError();
    });
}

}  // namespace mb
