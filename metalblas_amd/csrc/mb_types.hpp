// Element types, accumulator traits and the fused addmm epilogue shared by every kernel.
//
// Accumulation rules follow the reference profiles:
//   floats  (in, acc, out) = (T, fp32, T)            metalblas/float_dispatch.py:25-29
//   ints    accumulate in 32 bits (64 for int64) with wraparound, truncating store
//                                                    metalblas/integer_dispatch.py:13-19,
//                                                    shaders/int_gemm.h:134,147-150
//   complex products in fp32 (re/im), one rounding   metalblas/complex_dispatch.py:13-20,
//                                                    shaders/complex_pack.h:41-58
// Integer arithmetic is done in UNSIGNED types so wraparound is defined behaviour; the
// truncating store takes the low bits, which equals torch's int result modulo 2^bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mb {

// ---------------------------------------------------------------------------------------
// Storage types
// ---------------------------------------------------------------------------------------
struct alignas(8) c64_t { float re, im; };
struct alignas(4) c32_t { _Float16 re, im; };
using bf16_t = __bf16;
using f16_t = _Float16;

// fp32 complex accumulator
struct cf32 {
    float re, im;
};
__device__ __forceinline__ cf32 operator+(cf32 a, cf32 b) { return {a.re + b.re, a.im + b.im}; }
__device__ __forceinline__ cf32 operator*(cf32 a, cf32 b) {
    return {a.re * b.re - a.im * b.im, a.re * b.im + a.im * b.re};
}
__device__ __forceinline__ cf32 cmac(cf32 acc, cf32 a, cf32 b) {
    acc.re = __builtin_fmaf(a.re, b.re, acc.re);
    acc.re = __builtin_fmaf(-a.im, b.im, acc.re);
    acc.im = __builtin_fmaf(a.re, b.im, acc.im);
    acc.im = __builtin_fmaf(a.im, b.re, acc.im);
    return acc;
}

// ---------------------------------------------------------------------------------------
// Scalars handed to kernels (plain data, passed by value inside kernel arguments)
// ---------------------------------------------------------------------------------------
struct EpiScalars {
    float alpha_re, alpha_im, beta_re, beta_im;
    uint64_t alpha_u, beta_u;   // integer dtypes: two's-complement bits of alpha/beta
};

// ---------------------------------------------------------------------------------------
// Traits: acc type, widening load, narrowing store, multiply-accumulate, epilogue
// ---------------------------------------------------------------------------------------
template <class T> struct Tr;

template <> struct Tr<float> {
    using acc = float;
    static constexpr bool is_complex = false, is_int = false;
    __device__ static __forceinline__ acc up(float x, bool) { return x; }
    __device__ static __forceinline__ float down(acc v) { return v; }
    __device__ static __forceinline__ acc mac(acc s, acc a, acc b) { return __builtin_fmaf(a, b, s); }
    __device__ static __forceinline__ acc zero() { return 0.f; }
};
template <> struct Tr<f16_t> {
    using acc = float;
    static constexpr bool is_complex = false, is_int = false;
    __device__ static __forceinline__ acc up(f16_t x, bool) { return (float)x; }
    __device__ static __forceinline__ f16_t down(acc v) { return (f16_t)v; }
    __device__ static __forceinline__ acc mac(acc s, acc a, acc b) { return __builtin_fmaf(a, b, s); }
    __device__ static __forceinline__ acc zero() { return 0.f; }
};
template <> struct Tr<bf16_t> {
    using acc = float;
    static constexpr bool is_complex = false, is_int = false;
    __device__ static __forceinline__ acc up(bf16_t x, bool) { return (float)x; }
    __device__ static __forceinline__ bf16_t down(acc v) { return (bf16_t)v; }
    __device__ static __forceinline__ acc mac(acc s, acc a, acc b) { return __builtin_fmaf(a, b, s); }
    __device__ static __forceinline__ acc zero() { return 0.f; }
};
template <> struct Tr<c64_t> {
    using acc = cf32;
    static constexpr bool is_complex = true, is_int = false;
    __device__ static __forceinline__ acc up(c64_t x, bool conj) { return {x.re, conj ? -x.im : x.im}; }
    __device__ static __forceinline__ c64_t down(acc v) { return {v.re, v.im}; }
    __device__ static __forceinline__ acc mac(acc s, acc a, acc b) { return cmac(s, a, b); }
    __device__ static __forceinline__ acc zero() { return {0.f, 0.f}; }
};
template <> struct Tr<c32_t> {
    using acc = cf32;
    static constexpr bool is_complex = true, is_int = false;
    __device__ static __forceinline__ acc up(c32_t x, bool conj) {
        float im = (float)x.im;
        return {(float)x.re, conj ? -im : im};
    }
    __device__ static __forceinline__ c32_t down(acc v) { return {(f16_t)v.re, (f16_t)v.im}; }
    __device__ static __forceinline__ acc mac(acc s, acc a, acc b) { return cmac(s, a, b); }
    __device__ static __forceinline__ acc zero() { return {0.f, 0.f}; }
};

// Integer traits: S is the storage type, U the unsigned accumulator of the reference's
// ACC_T width (int -> 32 bit, long -> 64 bit).
template <class S, class U> struct TrInt {
    using acc = U;
    static constexpr bool is_complex = false, is_int = true;
    // sign- (or zero-) extend to the accumulator width, then reinterpret as unsigned
    __device__ static __forceinline__ acc up(S x, bool) {
        if constexpr (sizeof(U) == 8) return (U)(int64_t)x;
        else return (U)(int32_t)x;
    }
    __device__ static __forceinline__ S down(acc v) { return (S)v; }   // keeps the low bits
    __device__ static __forceinline__ acc mac(acc s, acc a, acc b) { return s + a * b; }
    __device__ static __forceinline__ acc zero() { return 0; }
};
template <> struct Tr<int8_t> : TrInt<int8_t, uint32_t> {};
template <> struct Tr<uint8_t> : TrInt<uint8_t, uint32_t> {
    __device__ static __forceinline__ acc up(uint8_t x, bool) { return (uint32_t)x; }
};
template <> struct Tr<int16_t> : TrInt<int16_t, uint32_t> {};
template <> struct Tr<int32_t> : TrInt<int32_t, uint32_t> {};
template <> struct Tr<int64_t> : TrInt<int64_t, uint64_t> {};

// Reduction helpers over accumulator types
__device__ __forceinline__ float acc_add(float a, float b) { return a + b; }
__device__ __forceinline__ cf32 acc_add(cf32 a, cf32 b) { return a + b; }
__device__ __forceinline__ uint32_t acc_add(uint32_t a, uint32_t b) { return a + b; }
__device__ __forceinline__ uint64_t acc_add(uint64_t a, uint64_t b) { return a + b; }

// wave64 butterfly sum (all lanes end with the total)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, 64);
    return v;
}
__device__ __forceinline__ uint64_t wave_sum(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
        lo = (uint32_t)__shfl_xor((int)lo, o, 64);
        hi = (uint32_t)__shfl_xor((int)hi, o, 64);
        v += ((uint64_t)hi << 32) | lo;
    }
    return v;
}
__device__ __forceinline__ cf32 wave_sum(cf32 v) { return {wave_sum(v.re), wave_sum(v.im)}; }

// ---------------------------------------------------------------------------------------
// Fused addmm epilogue: v = alpha*acc (if alpha_nz) + beta*bias (if beta_nz), computed in
// the scalar type (fp32 / complex fp32 / the unsigned accumulator), then ONE narrowing
// store.  Follows shaders/mb_epi.h:16-26 (floats/ints) and shaders/complex_pack.h:43-58
// (complex).  The bias is not dereferenced when beta_nz == 0, so a NaN bias cannot leak.
// ---------------------------------------------------------------------------------------
template <class T>
__device__ __forceinline__ typename Tr<T>::acc epi_apply(typename Tr<T>::acc v, const T *bias_elem,
                                                           const EpiScalars &s, int beta_nz,
                                                           int alpha_nz) {
    using A = typename Tr<T>::acc;
    if constexpr (Tr<T>::is_complex) {
        A out = {0.f, 0.f};
        if (alpha_nz) {
            out.re += s.alpha_re * v.re - s.alpha_im * v.im;
            out.im += s.alpha_re * v.im + s.alpha_im * v.re;
        }
        if (beta_nz) {
            A b = Tr<T>::up(*bias_elem, false);
            out.re += s.beta_re * b.re - s.beta_im * b.im;
            out.im += s.beta_re * b.im + s.beta_im * b.re;
        }
        return out;
    } else if constexpr (Tr<T>::is_int) {
        A out = 0;
        if (alpha_nz) out += (A)s.alpha_u * v;
        if (beta_nz) out += (A)s.beta_u * Tr<T>::up(*bias_elem, false);
        return out;
    } else {
        float out = 0.f;
        if (alpha_nz) out += s.alpha_re * v;
        if (beta_nz) out += s.beta_re * Tr<T>::up(*bias_elem, false);
        return out;
    }
}

// ---------------------------------------------------------------------------------------
// Kernel argument block shared by the GEMM / GEMV / fill / reduce kernels
// ---------------------------------------------------------------------------------------
struct GemmArgs {
    const void *a;
    const void *b;
    void *c;
    const void *bias;
    void *ws;   // split-K partial planes: acc-typed [splits][batch][M][N]
    int64_t a_rs, a_cs, a_bs;
    int64_t b_rs, b_cs, b_bs;
    int64_t c_rs, c_cs, c_bs;
    int64_t bias_rs, bias_cs, bias_bs;
    int32_t M, N, K, batch;
    int32_t conj_a, conj_b;
    int32_t epilogue, beta_nz, alpha_nz;
    int32_t splits;      // K slices (1 = none)
    int32_t k_chunk;     // K per slice
    int32_t swz;         // tile-order group log2
    int32_t nv;          // GEMV families: number of vectors (thin dim)
    int32_t vec_ok;      // GEMV families: vectorised loads allowed
    int32_t planes;      // write accumulator planes to ws even with one K slice (a later
                         // reduction kernel finishes the output)
    int32_t bias_vec;    // bias rows read as 4-element vectors (contiguous, 4-element aligned)
    int32_t persist;     // workgroups of a persistent grid that loops over tiles (0: one per tile)
    int32_t c_stream;    // output larger than the last-level cache: non-temporal output stores
    int32_t zblocks;     // grid z-blocks when fewer than the batch entries, each workgroup taking
                         // every zblocks-th entry in turn (0: one per entry, at most 65535)
    EpiScalars s;
};

// Final store of one output element: applies the epilogue when enabled.
template <class T>
__device__ __forceinline__ void store_out(const GemmArgs &g, T *c_elem, typename Tr<T>::acc v,
                                          int64_t bias_off) {
    if (g.epilogue) {
        const T *bp = g.beta_nz ? (const T *)g.bias + bias_off : nullptr;
        v = epi_apply<T>(v, bp, g.s, g.beta_nz, g.alpha_nz);
    }
    *c_elem = Tr<T>::down(v);
}

__host__ __device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace mb
