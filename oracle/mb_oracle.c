/*
 * mb_oracle.c — CPU restatement of the metalblas matmul semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the parity tests, the
 * __graft_entry__.smoke() check and bench.py's cpu_baseline leg compare the HIP kernels
 * against.  Nothing in the product (metalblas_amd/) loads or calls it.
 *
 * It takes the SAME descriptor as the GPU library (include/metalblas_amd.h), with HOST
 * pointers, and computes every element with a plain triple loop:
 *
 *   floats (bf16/fp16/fp32): inputs decoded exactly to double, products summed in double
 *       (the fp64 reference of the north star), epilogue alpha*acc + beta*bias in double,
 *       then one round-to-nearest-even to the output format.
 *       Reference: metalblas/float_dispatch.py:25-29 (fp32 accumulate, one rounding),
 *       shaders/mb_epi.h:16-26 (epilogue order, bias read only when beta != 0),
 *       tests/test_basic.py:37-42 (the reference's own oracle is a wider matmul).
 *   ints: exact two's-complement arithmetic modulo 2^64, then truncation to the output width.
 *       Modulo 2^bits this equals the reference's 32-bit (64-bit for int64) wraparound
 *       accumulate + truncating store: metalblas/integer_dispatch.py:13-19,
 *       shaders/int_gemm.h:134,147-150, tests/test_basic.py:27-34 (_wrap).
 *   complex (complex64/complex32): double-complex products, conj flags applied on read,
 *       complex epilogue alpha*P + beta*bias: shaders/complex_pack.h:41-58,
 *       shaders/cgemv_nt.h:34-56, tests/test_basic.py:40-41,60-64.
 *
 * Rounding helpers are written from the IEEE-754 binary16 / bfloat16 definitions
 * (1+10 / 1+7 fraction bits, exponent bias 15 / 127, round half to even).
 *
 * Optional out_f64 receives the unrounded result (batch*M*N doubles, or 2x for complex,
 * row-major, interleaved re/im) so tests can apply tolerances against the exact value.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../include/metalblas_amd.h"

/* ---------------- format helpers (from the definitions) ---------------- */

double mbo_bf16_to_double(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

double mbo_f16_to_double(uint16_t h) {
    const int sign = (h >> 15) & 1, exp = (h >> 10) & 0x1f, frac = h & 0x3ff;
    double v;
    if (exp == 0) v = ldexp((double)frac, -24);                 /* subnormal: frac * 2^-24 */
    else if (exp == 31) v = frac ? NAN : INFINITY;
    else v = ldexp((double)(1024 + frac), exp - 25);            /* (1.frac) * 2^(exp-15) */
    return sign ? -v : v;
}

/* Round x to a binary format with p significand bits, minimum normal exponent emin and
 * largest finite value maxv, ties to even.  Returns the rounded value as a double. */
static double round_format(double x, int p, int emin, double maxv) {
    if (x == 0.0 || isnan(x) || isinf(x)) return x;
    int e = ilogb(x);
    if (e < emin) e = emin;                     /* subnormal range: fixed quantum */
    const double scaled = ldexp(x, p - 1 - e);  /* exact: power-of-two scaling */
    double r = nearbyint(scaled);               /* default mode: round half to even */
    double y = ldexp(r, e - (p - 1));
    if (fabs(y) > maxv) return x > 0 ? INFINITY : -INFINITY;
    return y;
}

uint16_t mbo_double_to_bf16(double x) {
    if (isnan(x)) return 0x7fc0;
    const double y = round_format(x, 8, -126, 3.3895313892515355e38);
    float f = (float)y;   /* exact: y is representable in bf16, hence in fp32 */
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);
}

uint16_t mbo_double_to_f16(double x) {
    if (isnan(x)) return 0x7e00;
    const double y = round_format(x, 11, -14, 65504.0);
    const uint16_t sign = signbit(y) ? 0x8000 : 0;
    const double a = fabs(y);
    if (isinf(a)) return sign | 0x7c00;
    if (a == 0.0) return sign;
    int e = ilogb(a);
    if (e < -14) return sign | (uint16_t)ldexp(a, 24);                 /* subnormal */
    const uint16_t frac = (uint16_t)(ldexp(a, 10 - e) - 1024.0);
    return sign | (uint16_t)((e + 15) << 10) | frac;
}

float mbo_double_to_f32(double x) { return (float)x; /* C conversion: round to nearest even */ }

/* ---------------- element access ---------------- */

static int is_complex(int dt) { return dt == MB_DTYPE_C64 || dt == MB_DTYPE_C32; }
static int is_int(int dt) { return dt >= MB_DTYPE_I8 && dt <= MB_DTYPE_I64; }

static double load_real(int dt, const void *base, int64_t idx) {
    switch (dt) {
        case MB_DTYPE_F32: return (double)((const float *)base)[idx];
        case MB_DTYPE_F16: return mbo_f16_to_double(((const uint16_t *)base)[idx]);
        case MB_DTYPE_BF16: return mbo_bf16_to_double(((const uint16_t *)base)[idx]);
    }
    return 0.0;
}

static void load_complex(int dt, const void *base, int64_t idx, int conj, double *re, double *im) {
    if (dt == MB_DTYPE_C64) {
        const float *p = (const float *)base + 2 * idx;
        *re = p[0];
        *im = p[1];
    } else {
        const uint16_t *p = (const uint16_t *)base + 2 * idx;
        *re = mbo_f16_to_double(p[0]);
        *im = mbo_f16_to_double(p[1]);
    }
    if (conj) *im = -*im;
}

/* signed/unsigned integer element widened to its two's-complement 64-bit pattern */
static uint64_t load_int(int dt, const void *base, int64_t idx) {
    switch (dt) {
        case MB_DTYPE_I8: return (uint64_t)(int64_t)((const int8_t *)base)[idx];
        case MB_DTYPE_U8: return (uint64_t)((const uint8_t *)base)[idx];
        case MB_DTYPE_I16: return (uint64_t)(int64_t)((const int16_t *)base)[idx];
        case MB_DTYPE_I32: return (uint64_t)(int64_t)((const int32_t *)base)[idx];
        case MB_DTYPE_I64: return (uint64_t)((const int64_t *)base)[idx];
    }
    return 0;
}

static void store_int(int dt, void *base, int64_t idx, uint64_t v) {
    switch (dt) {
        case MB_DTYPE_I8: ((int8_t *)base)[idx] = (int8_t)(uint8_t)v; break;
        case MB_DTYPE_U8: ((uint8_t *)base)[idx] = (uint8_t)v; break;
        case MB_DTYPE_I16: ((int16_t *)base)[idx] = (int16_t)(uint16_t)v; break;
        case MB_DTYPE_I32: ((int32_t *)base)[idx] = (int32_t)(uint32_t)v; break;
        case MB_DTYPE_I64: ((int64_t *)base)[idx] = (int64_t)v; break;
    }
}

static void store_real(int dt, void *base, int64_t idx, double v) {
    switch (dt) {
        case MB_DTYPE_F32: ((float *)base)[idx] = mbo_double_to_f32(v); break;
        case MB_DTYPE_F16: ((uint16_t *)base)[idx] = mbo_double_to_f16(v); break;
        case MB_DTYPE_BF16: ((uint16_t *)base)[idx] = mbo_double_to_bf16(v); break;
    }
}

static void store_complex(int dt, void *base, int64_t idx, double re, double im) {
    if (dt == MB_DTYPE_C64) {
        float *p = (float *)base + 2 * idx;
        p[0] = (float)re;
        p[1] = (float)im;
    } else {
        uint16_t *p = (uint16_t *)base + 2 * idx;
        p[0] = mbo_double_to_f16(re);
        p[1] = mbo_double_to_f16(im);
    }
}

/* ---------------- the restatement ---------------- */

int mbo_gemm(const mb_gemm_desc *d, double *out_f64) {
    if (!d || d->dtype < 0 || d->dtype >= MB_DTYPE_COUNT) return MB_ERR_UNSUPPORTED_DTYPE;
    if (d->batch < 0 || d->M < 0 || d->N < 0 || d->K < 0) return MB_ERR_INVALID_ARG;
    const int dt = d->dtype;
    const int epi = d->epilogue != 0;
    const int bnz = epi && d->beta_nz, anz = epi ? d->alpha_nz != 0 : 1;
    const mb_matrix A = d->a, B = d->b, C = d->c, BI = d->bias;

    for (int64_t bz = 0; bz < d->batch; ++bz)
        for (int64_t m = 0; m < d->M; ++m)
            for (int64_t n = 0; n < d->N; ++n) {
                const int64_t ci = bz * C.batch_stride + m * C.row_stride + n * C.col_stride;
                const int64_t bi = bz * BI.batch_stride + m * BI.row_stride + n * BI.col_stride;
                const int64_t oi = (bz * d->M + m) * d->N + n;
                if (is_int(dt)) {
                    uint64_t acc = 0;
                    for (int64_t k = 0; k < d->K; ++k) {
                        const uint64_t x = load_int(dt, A.ptr, bz * A.batch_stride + m * A.row_stride + k * A.col_stride);
                        const uint64_t y = load_int(dt, B.ptr, bz * B.batch_stride + k * B.row_stride + n * B.col_stride);
                        acc += x * y;
                    }
                    uint64_t v = acc;
                    if (epi) {
                        v = 0;
                        if (anz) v += (uint64_t)d->alpha_int * acc;
                        if (bnz) v += (uint64_t)d->beta_int * load_int(dt, BI.ptr, bi);
                    }
                    store_int(dt, C.ptr, ci, v);
                    if (out_f64) out_f64[oi] = (double)(int64_t)v;
                } else if (is_complex(dt)) {
                    double sr = 0.0, si = 0.0;
                    for (int64_t k = 0; k < d->K; ++k) {
                        double ar, ai, br, bim;
                        load_complex(dt, A.ptr, bz * A.batch_stride + m * A.row_stride + k * A.col_stride, d->conj_a, &ar, &ai);
                        load_complex(dt, B.ptr, bz * B.batch_stride + k * B.row_stride + n * B.col_stride, d->conj_b, &br, &bim);
                        sr += ar * br - ai * bim;
                        si += ar * bim + ai * br;
                    }
                    double vr = sr, vi = si;
                    if (epi) {
                        vr = 0.0;
                        vi = 0.0;
                        if (anz) {
                            vr += d->alpha_re * sr - d->alpha_im * si;
                            vi += d->alpha_re * si + d->alpha_im * sr;
                        }
                        if (bnz) {
                            double xr, xi;
                            load_complex(dt, BI.ptr, bi, 0, &xr, &xi);
                            vr += d->beta_re * xr - d->beta_im * xi;
                            vi += d->beta_re * xi + d->beta_im * xr;
                        }
                    }
                    store_complex(dt, C.ptr, ci, vr, vi);
                    if (out_f64) {
                        out_f64[2 * oi] = vr;
                        out_f64[2 * oi + 1] = vi;
                    }
                } else {
                    double s = 0.0;
                    for (int64_t k = 0; k < d->K; ++k)
                        s += load_real(dt, A.ptr, bz * A.batch_stride + m * A.row_stride + k * A.col_stride) *
                             load_real(dt, B.ptr, bz * B.batch_stride + k * B.row_stride + n * B.col_stride);
                    double v = s;
                    if (epi) {
                        v = 0.0;
                        if (anz) v += d->alpha_re * s;
                        if (bnz) v += d->beta_re * load_real(dt, BI.ptr, bi);
                    }
                    store_real(dt, C.ptr, ci, v);
                    if (out_f64) out_f64[oi] = v;
                }
            }
    return MB_OK;
}
