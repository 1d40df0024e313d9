// Streaming GEMV kernels for the floating types (fp32 / fp16 / bf16), vector path only.
//
// Same two families as gemv.hip (dot: matrix rows contiguous along K, gemv_nt-like;
// axpy: matrix rows run along the output, gemv_t-like), written for HBM bandwidth:
//   * the matrix is read with 16-byte nontemporal loads (global_load_dwordx4 nt), so the
//     once-read stream does not evict the vectors from L1/L2;
//   * the inner loop is unrolled U times with all U*R loads issued before any arithmetic;
//   * no runtime branches inside the loop: the number of vectors is a template parameter,
//     vectors past the caller's count re-read the last vector (cache hit) and are dropped;
//   * dot reduces across the 64 lanes with a butterfly; axpy writes one fp32 partial plane
//     per K slice that the deterministic split-K reduction sums.
#include "launch.hpp"

// single-vector dot: one row per wave, 8 loads of 16 bytes in flight per lane (tuned on
// MI355X: 6.5 TB/s on a 16384 x 16384 bf16 matrix with a 2-blocks-per-CU persistent grid)
#ifndef DOT_R1
#define DOT_R1 1
#endif
#ifndef DOT_U1
#define DOT_U1 8
#endif

namespace mb {

namespace {

// 16 bytes of T -> fp32 multiply-accumulate helpers
template <class T> struct Chunk;
template <> struct Chunk<bf16_t> {
    static constexpr int V = 8;
    __device__ static __forceinline__ void unpack(uint4 u, float (&f)[8]) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
};
template <> struct Chunk<f16_t> {
    static constexpr int V = 8;
    __device__ static __forceinline__ void unpack(uint4 u, float (&f)[8]) {
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = (float)__builtin_bit_cast(f16_t, (uint16_t)(w[i] & 0xffffu));
            f[2 * i + 1] = (float)__builtin_bit_cast(f16_t, (uint16_t)(w[i] >> 16));
        }
    }
};
template <> struct Chunk<float> {
    static constexpr int V = 4;
    __device__ static __forceinline__ void unpack(uint4 u, float (&f)[4]) {
        f[0] = __uint_as_float(u.x);
        f[1] = __uint_as_float(u.y);
        f[2] = __uint_as_float(u.z);
        f[3] = __uint_as_float(u.w);
    }
};

template <class T> __device__ __forceinline__ void dot_chunk(float &acc, uint4 a, uint4 b) {
    constexpr int V = Chunk<T>::V;
    float fa[V], fb[V];
    Chunk<T>::unpack(a, fa);
    Chunk<T>::unpack(b, fb);
#pragma unroll
    for (int e = 0; e < V; ++e) acc = __builtin_fmaf(fa[e], fb[e], acc);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream(const uint4 *p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// dot family: Y(i, v) = sum_k Mat[i*ld + k] X(k, v); X contiguous along k (x_ks == 1).
// Persistent over row groups: wave w of the grid takes groups w, w + waves, ... so every
// wave streams whole rows and all CUs finish together.
template <class T, int NV, int R, int U>
__global__ __launch_bounds__(256) void k_dot_fast(GemvArgs g) {
    constexpr int V = Chunk<T>::V;
    const int lane = threadIdx.x & 63;
    const int nch = g.K / V;   // 16-byte chunks per row
    const int groups = (g.rows + R - 1) / R;
    const int nwaves = gridDim.x * 4;
    const int first = blockIdx.x * 4 + (threadIdx.x >> 6);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z)
    for (int grp = first; grp < groups; grp += nwaves) {
        const int row0 = grp * R;
        const T *mat = (const T *)g.mat + bz * g.mat_bs;
        const T *x = (const T *)g.x + bz * g.x_bs;
        const uint4 *mp[R];
        const uint4 *xp[NV];
#pragma unroll
        for (int r = 0; r < R; ++r) mp[r] = (const uint4 *)(mat + (int64_t)min(row0 + r, g.rows - 1) * g.mat_ld);
#pragma unroll
        for (int v = 0; v < NV; ++v) xp[v] = (const uint4 *)(x + (int64_t)min(v, g.nv - 1) * g.x_vs);
        float acc[R][NV];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int v = 0; v < NV; ++v) acc[r][v] = 0.f;

        int c = lane;
        for (; c + 64 * (U - 1) < nch; c += 64 * U) {
            uint4 m[U][R], xv[U][NV];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int r = 0; r < R; ++r) m[u][r] = ld_stream(mp[r] + c + 64 * u);
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int v = 0; v < NV; ++v) xv[u][v] = xp[v][c + 64 * u];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int v = 0; v < NV; ++v) dot_chunk<T>(acc[r][v], m[u][r], xv[u][v]);
        }
        for (; c < nch; c += 64) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint4 m = ld_stream(mp[r] + c);
#pragma unroll
                for (int v = 0; v < NV; ++v) dot_chunk<T>(acc[r][v], m, xp[v][c]);
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
                if (lane == ((r * NV + v) & 63) && v < g.nv && row < g.rows) {
                    float val = acc[r][v];
                    if (g.epilogue) {
                        const T *bp = g.beta_nz
                                          ? (const T *)g.bias + bz * g.bias_bs + row * g.bias_is + v * g.bias_vs
                                          : nullptr;
                        val = epi_apply<T>(val, bp, g.s, g.beta_nz, g.alpha_nz);
                    }
                    y[row * g.y_is + v * g.y_vs] = (T)val;
                }
            }
    }
}

// Single-vector dot, one workgroup per RW rows: thread t streams chunks t, t + 256, ... of
// each of its workgroup's rows (U loads per row in flight), so the whole grid reads W in
// near address order; the four wave partials meet in LDS.  Persistent over row groups.
template <class T, int RW, int U>
__global__ __launch_bounds__(256) void k_dot_wg(GemvArgs g) {
    constexpr int V = Chunk<T>::V;
    __shared__ float part[4][RW];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int nch = g.K / V;
    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z)
    for (int row0 = blockIdx.x * RW; row0 < g.rows; row0 += gridDim.x * RW) {
        const T *mat = (const T *)g.mat + bz * g.mat_bs;
        const uint4 *xp = (const uint4 *)((const T *)g.x + bz * g.x_bs);
        const uint4 *mp[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) mp[r] = (const uint4 *)(mat + (int64_t)min(row0 + r, g.rows - 1) * g.mat_ld);
        float acc[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = 0.f;
        int c = t;
        for (; c + 256 * (U - 1) < nch; c += 256 * U) {
            uint4 m[RW][U], xv[U];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int u = 0; u < U; ++u) m[r][u] = ld_stream(mp[r] + c + 256 * u);
#pragma unroll
            for (int u = 0; u < U; ++u) xv[u] = xp[c + 256 * u];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int u = 0; u < U; ++u) dot_chunk<T>(acc[r], m[r][u], xv[u]);
        }
        for (; c < nch; c += 256) {
            const uint4 xv = xp[c];
#pragma unroll
            for (int r = 0; r < RW; ++r) dot_chunk<T>(acc[r], ld_stream(mp[r] + c), xv);
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[r] = wave_sum(acc[r]);
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < RW; ++r) part[w][r] = acc[r];
        __syncthreads();
        if (t < RW && row0 + t < g.rows) {
            const int row = row0 + t;
            float val = (part[0][t] + part[1][t]) + (part[2][t] + part[3][t]);
            if (g.epilogue) {
                const T *bp = g.beta_nz ? (const T *)g.bias + bz * g.bias_bs + row * g.bias_is : nullptr;
                val = epi_apply<T>(val, bp, g.s, g.beta_nz, g.alpha_nz);
            }
            T *y = (T *)g.y + bz * g.y_bs;
            y[row * g.y_is] = (T)val;
        }
        __syncthreads();
    }
}

// complex64 single-vector dot on the k_dot_wg stream: each 16-byte chunk of a row holds two
// complex elements, multiplied into the row's (re, im) accumulators in fp32 with conj(W) and
// conj(x) as signs: y = sum (wr + i sa wi)(xr + i sb xi) = sum wr xr - sa sb wi xi
// + i (sb wr xi + sa wi xr).  Plain products only (the planner routes epilogues elsewhere).
template <int RW, int U>
__global__ __launch_bounds__(256) void k_cdot_wg(GemvArgs g) {
    __shared__ float part[4][RW][2];
    const float sa = g.conj_mat ? -1.f : 1.f, sb = g.conj_x ? -1.f : 1.f, sab = sa * sb;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int nch = g.K / 2;
    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z)
    for (int row0 = blockIdx.x * RW; row0 < g.rows; row0 += gridDim.x * RW) {
        const c64_t *mat = (const c64_t *)g.mat + bz * g.mat_bs;
        const uint4 *xp = (const uint4 *)((const c64_t *)g.x + bz * g.x_bs);
        const uint4 *mp[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) mp[r] = (const uint4 *)(mat + (int64_t)min(row0 + r, g.rows - 1) * g.mat_ld);
        float re[RW], im[RW];
#pragma unroll
        for (int r = 0; r < RW; ++r) re[r] = im[r] = 0.f;
        auto mac = [&](int r, uint4 m, uint4 x) {
            const float w0r = __uint_as_float(m.x), w0i = __uint_as_float(m.y);
            const float w1r = __uint_as_float(m.z), w1i = __uint_as_float(m.w);
            const float x0r = __uint_as_float(x.x), x0i = __uint_as_float(x.y);
            const float x1r = __uint_as_float(x.z), x1i = __uint_as_float(x.w);
            re[r] = __builtin_fmaf(w0r, x0r, re[r]);
            re[r] = __builtin_fmaf(w0i, -sab * x0i, re[r]);
            re[r] = __builtin_fmaf(w1r, x1r, re[r]);
            re[r] = __builtin_fmaf(w1i, -sab * x1i, re[r]);
            im[r] = __builtin_fmaf(w0r, sb * x0i, im[r]);
            im[r] = __builtin_fmaf(w0i, sa * x0r, im[r]);
            im[r] = __builtin_fmaf(w1r, sb * x1i, im[r]);
            im[r] = __builtin_fmaf(w1i, sa * x1r, im[r]);
        };
        int c = t;
        for (; c + 256 * (U - 1) < nch; c += 256 * U) {
            uint4 m[RW][U], xv[U];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int u = 0; u < U; ++u) m[r][u] = ld_stream(mp[r] + c + 256 * u);
#pragma unroll
            for (int u = 0; u < U; ++u) xv[u] = xp[c + 256 * u];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int u = 0; u < U; ++u) mac(r, m[r][u], xv[u]);
        }
        for (; c < nch; c += 256) {
            const uint4 xv = xp[c];
#pragma unroll
            for (int r = 0; r < RW; ++r) mac(r, ld_stream(mp[r] + c), xv);
        }
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            re[r] = wave_sum(re[r]);
            im[r] = wave_sum(im[r]);
        }
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                part[w][r][0] = re[r];
                part[w][r][1] = im[r];
            }
        __syncthreads();
        if (t < RW && row0 + t < g.rows) {
            const int row = row0 + t;
            c64_t v;
            v.re = (part[0][t][0] + part[1][t][0]) + (part[2][t][0] + part[3][t][0]);
            v.im = (part[0][t][1] + part[1][t][1]) + (part[2][t][1] + part[3][t][1]);
            ((c64_t *)g.y + bz * g.y_bs)[row * g.y_is] = v;
        }
        __syncthreads();
    }
}

// dot family with X stored k-major (X(k, v) at x[k*x_ks + v], NV values contiguous per k):
// the thin side of W @ X for a row-major X.  Each lane loads the V k-rows of X that match its
// 16-byte matrix chunk (V loads of NV elements) and reuses them for R matrix rows.
template <class T, int NV> struct alignas(NV * sizeof(T)) XRow {
    T e[NV];
};
template <class T, int NV, int R>
__global__ __launch_bounds__(256) void k_dot_xrow(GemvArgs g) {
    constexpr int V = Chunk<T>::V;
    const int lane = threadIdx.x & 63;
    const int nch = g.K / V;
    const int groups = (g.rows + R - 1) / R;
    const int nwaves = gridDim.x * 4;
    const int first = blockIdx.x * 4 + (threadIdx.x >> 6);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z)
    for (int grp = first; grp < groups; grp += nwaves) {
        const int row0 = grp * R;
        const T *mat = (const T *)g.mat + bz * g.mat_bs;
        const T *x = (const T *)g.x + bz * g.x_bs;
        const uint4 *mp[R];
#pragma unroll
        for (int r = 0; r < R; ++r) mp[r] = (const uint4 *)(mat + (int64_t)min(row0 + r, g.rows - 1) * g.mat_ld);
        float acc[R][NV];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int v = 0; v < NV; ++v) acc[r][v] = 0.f;
        for (int c = lane; c < nch; c += 64) {
            uint4 m[R];
#pragma unroll
            for (int r = 0; r < R; ++r) m[r] = ld_stream(mp[r] + c);
            XRow<T, NV> xr[V];
#pragma unroll
            for (int e = 0; e < V; ++e) xr[e] = *(const XRow<T, NV> *)(x + (int64_t)(c * V + e) * g.x_ks);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float f[V];
                Chunk<T>::unpack(m[r], f);
#pragma unroll
                for (int e = 0; e < V; ++e)
#pragma unroll
                    for (int v = 0; v < NV; ++v) acc[r][v] = __builtin_fmaf(f[e], (float)xr[e].e[v], acc[r][v]);
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
                if (lane == ((r * NV + v) & 63) && row < g.rows) {
                    float val = acc[r][v];
                    if (g.epilogue) {
                        const T *bp = g.beta_nz
                                          ? (const T *)g.bias + bz * g.bias_bs + row * g.bias_is + v * g.bias_vs
                                          : nullptr;
                        val = epi_apply<T>(val, bp, g.s, g.beta_nz, g.alpha_nz);
                    }
                    y[row * g.y_is + v * g.y_vs] = (T)val;
                }
            }
    }
}

// axpy family: Y(v, i) = sum_k X(v, k) Mat[k*ld + i]; each wave owns 64*VEC columns (VEC
// elements per lane, one 16-byte load per row) and the K slice blockIdx.y.
template <class T, int NV, int U>
__global__ __launch_bounds__(256) void k_axpy_fast(GemvArgs g) {
    constexpr int V = Chunk<T>::V;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wcol = (blockIdx.x * 4 + w) * 64 * V;
    if (wcol >= g.rows) return;
    const int col0 = wcol + lane * V;
    const bool live = col0 < g.rows;
    const int colc = live ? col0 : wcol;
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const T *mat = (const T *)g.mat + bz * g.mat_bs + colc;
        const T *x = (const T *)g.x + bz * g.x_bs;
        float acc[NV][V];
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
            for (int e = 0; e < V; ++e) acc[v][e] = 0.f;
        int64_t xvo[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) xvo[v] = (int64_t)min(v, g.nv - 1) * g.x_vs;

        int k = kbeg;
        for (; k + U <= kend; k += U) {
            uint4 m[U];
#pragma unroll
            for (int u = 0; u < U; ++u) m[u] = ld_stream((const uint4 *)(mat + (int64_t)(k + u) * g.mat_ld));
            float xs[U][NV];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int v = 0; v < NV; ++v) xs[u][v] = (float)x[(int64_t)(k + u) * g.x_ks + xvo[v]];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float f[V];
                Chunk<T>::unpack(m[u], f);
#pragma unroll
                for (int v = 0; v < NV; ++v)
#pragma unroll
                    for (int e = 0; e < V; ++e) acc[v][e] = __builtin_fmaf(xs[u][v], f[e], acc[v][e]);
            }
        }
        for (; k < kend; ++k) {
            const uint4 m = ld_stream((const uint4 *)(mat + (int64_t)k * g.mat_ld));
            float f[V];
            Chunk<T>::unpack(m, f);
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                const float xe = (float)x[(int64_t)k * g.x_ks + xvo[v]];
#pragma unroll
                for (int e = 0; e < V; ++e) acc[v][e] = __builtin_fmaf(xe, f[e], acc[v][e]);
            }
        }
        if (!live) continue;
        if (g.splits > 1) {
            float *ws = (float *)g.ws;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                if (v >= g.nv) continue;
                float *dst = ws + (((int64_t)ks * g.batch + bz) * g.nv + v) * g.rows + col0;
                if constexpr (V == 8) {
                    *(float4 *)dst = make_float4(acc[v][0], acc[v][1], acc[v][2], acc[v][3]);
                    *(float4 *)(dst + 4) = make_float4(acc[v][4], acc[v][5], acc[v][6], acc[v][7]);
                } else {
                    *(float4 *)dst = make_float4(acc[v][0], acc[v][1], acc[v][2], acc[v][3]);
                }
            }
        } else {
            T *y = (T *)g.y + bz * g.y_bs;
#pragma unroll
            for (int v = 0; v < NV; ++v) {
                if (v >= g.nv) continue;
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const int col = col0 + e;
                    float val = acc[v][e];
                    if (g.epilogue) {
                        const T *bp = g.beta_nz
                                          ? (const T *)g.bias + bz * g.bias_bs + col * g.bias_is + v * g.bias_vs
                                          : nullptr;
                        val = epi_apply<T>(val, bp, g.s, g.beta_nz, g.alpha_nz);
                    }
                    y[col * g.y_is + v * g.y_vs] = (T)val;
                }
            }
        }
    }
}

// axpy family, one vector: workgroup-wide column bands.  A workgroup owns 256 * CH chunks of V
// columns (thread t: chunks t + 256 j) and the K slice blockIdx.y, so each row of the slice is
// read as one contiguous span of 4 KiB * CH, with CH * U 16-byte loads in flight per thread.
// Measured on MI355X, 16384^2 bf16 with 128 K slices (one workgroup per CU): CH = 4, U = 2
// streams the matrix at 7.1 TB/s, against 6.6 TB/s for the 64-lane wave bands of k_axpy_fast.
template <class T, int CH, int U>
__global__ __launch_bounds__(256) void k_axpy_band(GemvArgs g) {
    constexpr int V = Chunk<T>::V;
    const int t = threadIdx.x;
    const int band0 = blockIdx.x * 256 * V * CH;   // < g.rows: the grid has ceil(rows / band) columns
    int col[CH], colc[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        col[j] = band0 + (t + 256 * j) * V;
        colc[j] = col[j] < g.rows ? col[j] : band0;   // columns past the edge re-read the band start
    }
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const T *mat = (const T *)g.mat + bz * g.mat_bs;
        const T *x = (const T *)g.x + bz * g.x_bs;
        float acc[CH][V];
#pragma unroll
        for (int j = 0; j < CH; ++j)
#pragma unroll
            for (int e = 0; e < V; ++e) acc[j][e] = 0.f;

        int k = kbeg;
        for (; k + U <= kend; k += U) {
            uint4 m[U][CH];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int j = 0; j < CH; ++j)
                    m[u][j] = ld_stream((const uint4 *)(mat + (int64_t)(k + u) * g.mat_ld + colc[j]));
            float xs[U];
#pragma unroll
            for (int u = 0; u < U; ++u) xs[u] = (float)x[(int64_t)(k + u) * g.x_ks];
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    float f[V];
                    Chunk<T>::unpack(m[u][j], f);
#pragma unroll
                    for (int e = 0; e < V; ++e) acc[j][e] = __builtin_fmaf(xs[u], f[e], acc[j][e]);
                }
        }
        for (; k < kend; ++k) {
            const float xe = (float)x[(int64_t)k * g.x_ks];
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                float f[V];
                Chunk<T>::unpack(ld_stream((const uint4 *)(mat + (int64_t)k * g.mat_ld + colc[j])), f);
#pragma unroll
                for (int e = 0; e < V; ++e) acc[j][e] = __builtin_fmaf(xe, f[e], acc[j][e]);
            }
        }
        if (g.splits > 1) {
            float *ws = (float *)g.ws + ((int64_t)ks * g.batch + bz) * g.rows;   // nv == 1
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                if (col[j] >= g.rows) continue;
#pragma unroll
                for (int e = 0; e < V; e += 4)
                    *(float4 *)(ws + col[j] + e) = make_float4(acc[j][e], acc[j][e + 1], acc[j][e + 2], acc[j][e + 3]);
            }
        } else {
            T *y = (T *)g.y + bz * g.y_bs;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                if (col[j] >= g.rows) continue;
#pragma unroll
                for (int e = 0; e < V; ++e) {
                    const int c = col[j] + e;
                    float val = acc[j][e];
                    if (g.epilogue) {
                        const T *bp = g.beta_nz ? (const T *)g.bias + bz * g.bias_bs + c * g.bias_is : nullptr;
                        val = epi_apply<T>(val, bp, g.s, g.beta_nz, g.alpha_nz);
                    }
                    y[c * g.y_is] = (T)val;
                }
            }
        }
    }
}
constexpr int kBandU = 2;
// 16-byte chunks per thread of the column band: 4 (256 threads x 4 chunks = 16 KiB of each
// row) where the rows are that wide, else the widest band that does not overhang the row, so
// narrow matrices get more column blocks instead of re-read columns
__host__ __device__ inline int band_ch(int64_t rows, int vec) {
    return rows >= 256 * vec * 4 ? 4 : (rows >= 256 * vec * 2 ? 2 : 1);
}

template <class T, int NV> hipError_t dot_xrow_launch(const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    constexpr int R = NV >= 16 ? 2 : (NV >= 8 ? 4 : 8);
    const int groups = cdiv(g.rows, R);
    int blocks = cdiv(groups, 4);
    if (g.grid_cap > 0 && blocks > g.grid_cap) blocks = g.grid_cap;
    dim3 grid(blocks, 1, g.batch < 65535 ? g.batch : 65535), block(256);
    if (shape) *shape = {grid, block};
    hipLaunchKernelGGL((k_dot_xrow<T, NV, R>), grid, block, 0, st, g);
    return hipGetLastError();
}

template <class T, int NV> hipError_t dot_fast_launch(const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    if constexpr (NV > 1) {
        if (g.x_row) return dot_xrow_launch<T, NV>(g, st, shape);
    } else {
        // one vector: workgroup-wide row streams (measured on MI355X, 16384^2 bf16: 77 us,
        // 6.9 TB/s, against 82 us for a row per wave), 2 rows x 4 loads in flight per thread,
        // 4 workgroups per CU
        constexpr int RW = 2, U = 4;
        int blocks = cdiv(g.rows, RW);
        const int cap = g.grid_cap > 0 ? 2 * g.grid_cap : 0;
        if (cap > 0 && blocks > cap) blocks = cap;
        dim3 grid(blocks, 1, g.batch < 65535 ? g.batch : 65535), block(256);
        if (shape) *shape = {grid, block};
        hipLaunchKernelGGL((k_dot_wg<T, RW, U>), grid, block, 0, st, g);
        return hipGetLastError();
    }
    constexpr int R = NV == 1 ? DOT_R1 : (NV <= 4 ? 4 : (NV == 8 ? 4 : 2));
    constexpr int U = NV == 1 ? DOT_U1 : (NV <= 4 ? 2 : 1);
    const int groups = cdiv(g.rows, R);
    int blocks = cdiv(groups, 4);
    if (g.grid_cap > 0 && blocks > g.grid_cap) blocks = g.grid_cap;
    dim3 grid(blocks, 1, g.batch < 65535 ? g.batch : 65535), block(256);
    if (shape) *shape = {grid, block};
    hipLaunchKernelGGL((k_dot_fast<T, NV, R, U>), grid, block, 0, st, g);
    return hipGetLastError();
}

template <class T, int NV> hipError_t axpy_fast_launch(const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    if constexpr (NV == 1) {
        const int ch = band_ch(g.rows, Chunk<T>::V);
        const int band = 256 * Chunk<T>::V * ch;
        dim3 grid(cdiv(g.rows, band), g.splits, g.batch < 65535 ? g.batch : 65535), block(256);
        if (shape) *shape = {grid, block};
        if (ch == 4)
            hipLaunchKernelGGL((k_axpy_band<T, 4, kBandU>), grid, block, 0, st, g);
        else if (ch == 2)
            hipLaunchKernelGGL((k_axpy_band<T, 2, kBandU>), grid, block, 0, st, g);
        else
            hipLaunchKernelGGL((k_axpy_band<T, 1, kBandU>), grid, block, 0, st, g);
        return hipGetLastError();
    }
    constexpr int U = NV <= 2 ? 8 : 4;
    const int waves = cdiv(g.rows, 64 * Chunk<T>::V);
    dim3 grid(cdiv(waves, 4), g.splits, g.batch < 65535 ? g.batch : 65535), block(256);
    if (shape) *shape = {grid, block};
    hipLaunchKernelGGL((k_axpy_fast<T, NV, U>), grid, block, 0, st, g);
    return hipGetLastError();
}

template <class T, template <class, int> class L>
hipError_t by_nv(const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    const int b = gemv_nv_bucket(g.nv);
    switch (b) {
        case 1: return L<T, 1>::run(g, st, shape);
        case 2: return L<T, 2>::run(g, st, shape);
        case 4: return L<T, 4>::run(g, st, shape);
        case 8: return L<T, 8>::run(g, st, shape);
        case 16: return L<T, 16>::run(g, st, shape);
    }
    return hipErrorInvalidValue;
}
template <class T, int NV> struct DotL {
    static hipError_t run(const GemvArgs &g, hipStream_t st, LaunchShape *s) { return dot_fast_launch<T, NV>(g, st, s); }
};
template <class T, int NV> struct AxpyL {
    static hipError_t run(const GemvArgs &g, hipStream_t st, LaunchShape *s) { return axpy_fast_launch<T, NV>(g, st, s); }
};

}  // namespace

bool gemv_fast_dtype(int dt) { return dt == F32 || dt == F16 || dt == BF16; }
int gemv_fast_vec(int dt) { return 16 / dtype_size(dt); }
int gemv_axpy_band_cols(int dt, int nv, int64_t rows) {
    const int vec = 16 / dtype_size(dt);
    return nv == 1 ? 256 * vec * band_ch(rows, vec) : 0;
}

hipError_t launch_gemv_dot_fast(int dt, const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    if (dt == C64) {   // one vector, no epilogue (plan_gemv): the k_dot_wg stream
        if (g.nv != 1 || g.epilogue) return hipErrorInvalidValue;
        constexpr int RW = 2, U = 4;
        int blocks = cdiv(g.rows, RW);
        const int cap = g.grid_cap > 0 ? 2 * g.grid_cap : 0;
        if (cap > 0 && blocks > cap) blocks = cap;
        dim3 grid(blocks, 1, g.batch < 65535 ? g.batch : 65535), block(256);
        if (shape) *shape = {grid, block};
        hipLaunchKernelGGL((k_cdot_wg<RW, U>), grid, block, 0, st, g);
        return hipGetLastError();
    }
    switch (dt) {
        case F32: return by_nv<float, DotL>(g, st, shape);
        case F16: return by_nv<f16_t, DotL>(g, st, shape);
        case BF16: return by_nv<bf16_t, DotL>(g, st, shape);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_axpy_fast(int dt, const GemvArgs &g, hipStream_t st, LaunchShape *shape) {
    switch (dt) {
        case F32: return by_nv<float, AxpyL>(g, st, shape);
        case F16: return by_nv<f16_t, AxpyL>(g, st, shape);
        case BF16: return by_nv<bf16_t, AxpyL>(g, st, shape);
    }
    return hipErrorInvalidValue;
}

}  // namespace mb
