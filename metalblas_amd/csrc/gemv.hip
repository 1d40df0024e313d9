// Bandwidth-bound matrix-vector families (one or a few vectors).
//
//   dot  : Y(i, v) = sum_k Mat[i*ld + k] * X(k, v)   matrix rows contiguous along K
//          (the reference's gemv_nt, shaders/gemv_nt.h:16-101, and the TRANS_B form of
//          gemv_bt, shaders/gemv_bt.h:78-180)
//   axpy : Y(v, i) = sum_k X(v, k) * Mat[k*ld + i]   matrix rows run along the output
//          (the reference's gemv_t, shaders/gemv_t.h:15-99, and gemv_bt, :181-267)
//
// wave64 design: the dot family gives each wave R rows and streams them with 16-byte loads,
// re-using every loaded X chunk for the R rows, and reduces with a butterfly over the 64
// lanes.  The axpy family gives each wave 64*V contiguous output columns and a K slice; the
// grid's y dimension splits K so that >= 8 waves per CU are resident even for a single
// vector, and the slices are summed by the deterministic split-K reduction kernel.
#include "launch.hpp"

namespace mb {

namespace {

template <class T, int V> struct alignas(V * sizeof(T)) VecT {
    T e[V];
};

// ------------------------------------------------------------------------------------
// dot family
// ------------------------------------------------------------------------------------
template <class T, int NV, int R, bool VEC>
__global__ __launch_bounds__(256) void k_gemv_dot(GemvArgs g) {
    using A = typename Tr<T>::acc;
    constexpr int V = VEC ? 16 / (int)sizeof(T) : 1;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + w) * R;
    if (row0 >= g.rows) return;   // whole wave leaves; no block-level barrier below

    int rowc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rowc[r] = min(row0 + r, g.rows - 1);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const T *mat = (const T *)g.mat + bz * g.mat_bs;
        const T *x = (const T *)g.x + bz * g.x_bs;
        A acc[R][NV];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int v = 0; v < NV; ++v) acc[r][v] = Tr<T>::zero();

        if constexpr (VEC) {
#pragma unroll 2
            for (int k = lane * V; k < g.K; k += 64 * V) {
                VecT<T, V> xv[NV], mv[R];
#pragma unroll
                for (int v = 0; v < NV; ++v)
                    if (v < g.nv) xv[v] = *(const VecT<T, V> *)(x + v * g.x_vs + k);
#pragma unroll
                for (int r = 0; r < R; ++r)
                    mv[r] = *(const VecT<T, V> *)(mat + rowc[r] * g.mat_ld + k);
#pragma unroll
                for (int e = 0; e < V; ++e)
#pragma unroll
                    for (int v = 0; v < NV; ++v) {
                        if (v >= g.nv) continue;
                        const A xe = Tr<T>::up(xv[v].e[e], g.conj_x);
#pragma unroll
                        for (int r = 0; r < R; ++r)
                            acc[r][v] = Tr<T>::mac(acc[r][v], Tr<T>::up(mv[r].e[e], g.conj_mat), xe);
                    }
            }
        } else {
            for (int k = lane; k < g.K; k += 64) {
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    if (v >= g.nv) continue;
                    const A xe = Tr<T>::up(x[k * g.x_ks + v * g.x_vs], g.conj_x);
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        acc[r][v] = Tr<T>::mac(acc[r][v],
                                               Tr<T>::up(mat[rowc[r] * g.mat_ld + k], g.conj_mat), xe);
                }
            }
        }

#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int v = 0; v < NV; ++v) acc[r][v] = wave_sum(acc[r][v]);

        T *y = (T *)g.y + bz * g.y_bs;
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const int row = row0 + r;
                if (lane == r * NV + v && v < g.nv && row < g.rows) {
                    A val = acc[r][v];
                    if (g.epilogue) {
                        const T *bp = g.beta_nz
                                          ? (const T *)g.bias + bz * g.bias_bs + row * g.bias_is + v * g.bias_vs
                                          : nullptr;
                        val = epi_apply<T>(val, bp, g.s, g.beta_nz, g.alpha_nz);
                    }
                    y[row * g.y_is + v * g.y_vs] = Tr<T>::down(val);
                }
            }
    }
}

// ------------------------------------------------------------------------------------
// axpy family
// ------------------------------------------------------------------------------------
template <class T, int NV, int V>
__global__ __launch_bounds__(256) void k_gemv_axpy(GemvArgs g) {
    using A = typename Tr<T>::acc;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col0 = ((blockIdx.x * 4 + w) * 64 + lane) * V;
    if ((blockIdx.x * 4 + w) * 64 * V >= g.rows) return;   // whole wave out of range
    const bool live = col0 < g.rows;
    const int colc = live ? col0 : 0;
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const T *mat = (const T *)g.mat + bz * g.mat_bs;
        const T *x = (const T *)g.x + bz * g.x_bs;
        A acc[NV][V];
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
            for (int e = 0; e < V; ++e) acc[v][e] = Tr<T>::zero();

#pragma unroll 4
        for (int k = kbeg; k < kend; ++k) {
            VecT<T, V> mv = *(const VecT<T, V> *)(mat + k * g.mat_ld + colc);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                if (v >= g.nv) continue;
                const A xe = Tr<T>::up(x[k * g.x_ks + v * g.x_vs], g.conj_x);
#pragma unroll
                for (int e = 0; e < V; ++e)
                    acc[v][e] = Tr<T>::mac(acc[v][e], Tr<T>::up(mv.e[e], g.conj_mat), xe);
            }
        }
        if (!live) continue;

        if (g.splits > 1) {
            A *ws = (A *)g.ws;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                if (v >= g.nv) continue;
                A *dst = ws + (((int64_t)ks * g.batch + bz) * g.nv + v) * g.rows + col0;
#pragma unroll
                for (int e = 0; e < V; ++e) dst[e] = acc[v][e];
            }
        } else {
            T *y = (T *)g.y + bz * g.y_bs;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                if (v >= g.nv) continue;
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const int col = col0 + e;
                    A val = acc[v][e];
                    if (g.epilogue) {
                        const T *bp = g.beta_nz
                                          ? (const T *)g.bias + bz * g.bias_bs + col * g.bias_is + v * g.bias_vs
                                          : nullptr;
                        val = epi_apply<T>(val, bp, g.s, g.beta_nz, g.alpha_nz);
                    }
                    y[col * g.y_is + v * g.y_vs] = Tr<T>::down(val);
                }
            }
        }
    }
}

template <class T> constexpr int axpy_vec(int nv) {
    int v = 16 / (int)sizeof(T);
    const int cap = nv >= 1 ? 64 / nv : 64;
    if (v > cap) v = cap;
    return v < 1 ? 1 : v;
}

template <class T, int NV> hipError_t dot_launch(const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    constexpr int R = NV <= 4 ? 4 : (NV == 8 ? 2 : 1);
    const int waves = cdiv(g.rows, R);
    dim3 grid(cdiv(waves, 4), 1, g.batch < 65535 ? g.batch : 65535), block(256);
    if (shape) *shape = {grid, block};
    if (g.vec_ok)
        hipLaunchKernelGGL((k_gemv_dot<T, NV, R, true>), grid, block, 0, st, g);
    else
        hipLaunchKernelGGL((k_gemv_dot<T, NV, R, false>), grid, block, 0, st, g);
    return hipGetLastError();
}

template <class T, int NV> hipError_t axpy_launch(const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    constexpr int VV = axpy_vec<T>(NV);
    const int V = g.vec_ok ? VV : 1;
    const int waves = cdiv(g.rows, 64 * V);
    dim3 grid(cdiv(waves, 4), g.splits, g.batch < 65535 ? g.batch : 65535), block(256);
    if (shape) *shape = {grid, block};
    if (g.vec_ok)
        hipLaunchKernelGGL((k_gemv_axpy<T, NV, VV>), grid, block, 0, st, g);
    else
        hipLaunchKernelGGL((k_gemv_axpy<T, NV, 1>), grid, block, 0, st, g);
    return hipGetLastError();
}

}  // namespace

int gemv_nv_bucket(int nv) {
    if (nv <= 1) return 1;
    if (nv <= 2) return 2;
    if (nv <= 4) return 4;
    if (nv <= 8) return 8;
    if (nv <= 16) return 16;
    return 0;
}

int gemv_axpy_vec(int dt, int nv) {
    const int b = gemv_nv_bucket(nv);
    int v = 16 / dtype_size(dt);
    const int cap = b >= 1 ? 64 / b : 64;
    if (v > cap) v = cap;
    return v < 1 ? 1 : v;
}

hipError_t launch_gemv_dot(int dt, const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    const int b = gemv_nv_bucket(g.nv);
    return with_dtype(dt, [&]<class T>() {
        switch (b) {
            case 1: return dot_launch<T, 1>(g, st, shape);
            case 2: return dot_launch<T, 2>(g, st, shape);
            case 4: return dot_launch<T, 4>(g, st, shape);
            case 8: return dot_launch<T, 8>(g, st, shape);
            case 16: return dot_launch<T, 16>(g, st, shape);
        }
        return hipErrorInvalidValue;
    });
}

hipError_t launch_gemv_axpy(int dt, const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    const int b = gemv_nv_bucket(g.nv);
    return with_dtype(dt, [&]<class T>() {
        switch (b) {
            case 1: return axpy_launch<T, 1>(g, st, shape);
            case 2: return axpy_launch<T, 2>(g, st, shape);
            case 4: return axpy_launch<T, 4>(g, st, shape);
            case 8: return axpy_launch<T, 8>(g, st, shape);
            case 16: return axpy_launch<T, 16>(g, st, shape);
        }
        return hipErrorInvalidValue;
    });
}

}  // namespace mb
