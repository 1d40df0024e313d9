// Matrix-core GEMM for 16-bit inputs (bf16 / fp16) and 8-bit integers (int8 / uint8) on
// gfx950, fed by LDS-direct loads.  A stage is always 128 bytes of K per M/N index: 64 bf16 /
// fp16 (v_mfma_f32_32x32x16, 4 k-steps of 16) or 128 int8 (v_mfma_i32_32x32x32_i8, 4 k-steps
// of 32), so the LDS geometry, the swizzles of K-contiguous operands and the pipeline are
// shared; only the transposing read of M/N-contiguous operands differs
// (ds_read_b64_tr_b16 vs ds_read_b64_tr_b8).
//
// Differences from the register-staged matrix-core template (mfma_gemm.hpp):
//   * Operand tiles go from global memory straight into LDS with buffer_load_dwordx4 ... lds
//     (64 lanes x 16 bytes = 1 KiB per instruction, lane-contiguous in LDS).  No staging
//     registers and no register transposes: the LDS layout is chosen by giving each lane the
//     global chunk that belongs at its LDS slot.  Rows past the matrix edge use a buffer
//     offset beyond the resource's range, which the hardware turns into zeros.  The per-lane
//     offsets are loop invariant; the K advance of each stage travels in the uniform
//     soffset operand.
//   * Operands contiguous along K are stored K-major (one 128-byte row per M/N index,
//     16-byte chunks XOR-swizzled by (row & 7) ^ ((row >> 3) & 3), periodic in 32 rows) and
//     read as 16-byte fragments (ds_read_b128).
//   * Operands contiguous along M/N are stored M/N-major (one row per k) and read with
//     ds_read_b64_tr_b16: each 16-lane group transposes a 4 (k) x 16 (m/n) block, so two
//     such reads give a lane the 8 consecutive k of one column that the 32x32x16 MFMA
//     expects.  Chunks are XOR-swizzled by k % 4 with {0, 4, 10, 14}, which keeps a 16-lane
//     and a 32-lane slice of one read on distinct 16-byte bank groups.
//   * Stage pipeline: two LDS buffers; the loads of stage kt+2 are issued right after the
//     barrier that retires stage kt, and the MFMAs of the last k-step of stage kt are issued
//     after that barrier so they cover the latency of the first fragment reads of kt+1.
//   * C^T = B^T A^T product for 4-wide output stores, fused epilogue, split-K partial planes,
//     batching and the XCD-aware tile order are shared with mfma_gemm.hpp.
#pragma once

#include "launch.hpp"

namespace mb {
namespace m16 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
#define MB_LDS __attribute__((address_space(3)))

constexpr uint32_t kOOB = 0x80000000u;   // buffer offset that is always out of range

// One LDS-direct load: 64 lanes x 16 bytes from rsrc + voffset + soffset into LDS at lds_addr
// (+ 16 * lane), written as inline assembly.  The compiler does not model the LDS write of an
// asm statement, so it adds no wait of its own before later LDS reads; with the intrinsic
// form it waits for EVERY outstanding LDS-direct load before the first LDS read of a stage,
// which exposes the whole global-load latency of the prefetched stage once per stage.  The
// kernel instead waits for its own loads right before the barrier that publishes a stage,
// when only that stage's loads (and one L2 prefetch) are in flight.  M0 carries the LDS
// address.
//
// The compiler's hazard recognizer does not see the VMEM instruction inside the asm, so the
// asm supplies its own wait states: on gfx950 a VMEM instruction that reads an SGPR written
// by a VALU instruction needs 5 of them (the compiler emits `s_nop 4` for its own buffer
// loads).  Such writes do occur right before these loads: SGPR spill reloads are
// v_readlane_b32, and `readfirstlane` results.  With fewer wait states the load may read the
// SGPR's previous value as its resource or offset, i.e. an arbitrary address.  `s_nop 4` also
// covers the 1-wait-state M0 write -> LDS-DMA hazard.
// NT: a non-temporal load, for operands that are streamed from HBM once (the thin and deep-K
// products): their lines are not kept in the caches for reuse.
template <bool NT = false>
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset, int soffset) {
    if constexpr (NT)
        asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds"
                     :
                     : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds_addr)
                     : "memory");
    else
        asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                     :
                     : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds_addr)
                     : "memory");
}
__device__ __forceinline__ void vm_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// All but the most recent load have completed (loads retire in issue order).
__device__ __forceinline__ void vm_wait_but_one() { asm volatile("s_waitcnt vmcnt(1)" ::: "memory"); }

// L2 prefetch of one 128-byte line per lane: a dword LDS-direct load into a junk LDS area, so
// no VGPR is written behind the compiler's back.  Out-of-range offsets load nothing.  Same
// 5 wait states as dma16.
__device__ __forceinline__ void pf_line(i32x4 rsrc, uint32_t lds_addr, uint32_t voffset, int soffset) {
    asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, %2 offen lds"
                 :
                 : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds_addr)
                 : "memory");
}
constexpr int kPfDist = 3;   // stages between a line's L2 prefetch and its LDS-direct load

// Byte offset (from the operand tile's first element) of 128-byte line `idx` of one stage
// (128 bytes of K) of a ROWS-wide operand tile with ES-byte elements, or kOOB.  K-contiguous
// operands have one line per row; M/N-contiguous ones have ROWS * ES / 128 lines per k.
// Every stage has ROWS lines.
template <int ROWS, bool KC, int ES>
__device__ __forceinline__ uint32_t pf_line_offset(int idx, int64_t ld, int rows_left, int k_left) {
    if constexpr (KC) {
        if (idx >= ROWS || idx >= rows_left) return kOOB;
        return (uint32_t)((int64_t)idx * ld * ES);
    } else {
        constexpr int LPR = ROWS * ES / 128;
        constexpr int EPL = 128 / ES;   // elements per line
        const int r = idx / LPR, c = idx % LPR;
        if (r >= 128 / ES || r >= k_left || c * EPL >= rows_left) return kOOB;
        return (uint32_t)(((int64_t)r * ld + c * EPL) * ES);
    }
}
template <int BM, int BN, bool A_KC, bool B_KC, int ES>
__device__ __forceinline__ uint32_t pf_assign(int wave, int lane, int tm, int tn, int64_t lda, int64_t ldb,
                                              int rows_a, int rows_b, int k_left) {
    if (wave == 0 && lane < BM / 4)
        return pf_line_offset<BM, A_KC, ES>((tn & 3) * (BM / 4) + lane, lda, rows_a, k_left);
    if (wave == 1 && lane < BN / 8)
        return pf_line_offset<BN, B_KC, ES>((tm & 7) * (BN / 8) + lane, ldb, rows_b, k_left);
    return kOOB;
}

struct __attribute__((packed)) BufRes {
    const void *base;
    uint32_t range;
    uint32_t config;
};
__device__ __forceinline__ i32x4 make_rsrc(const void *base) {
    BufRes r{base, 0x7fffffffu, 0x00020000u};
    return __builtin_bit_cast(i32x4, r);
}

// Accumulator block of one 32 x 32 MFMA: fp32 for the float types, int32 (wrapping) for int8.
template <class T> struct AccV { using type = f32x16; };
template <> struct AccV<int8_t> { using type = i32x16; };
template <> struct AccV<uint8_t> { using type = i32x16; };

template <class T> __device__ __forceinline__ void mma16(typename AccV<T>::type &c, uint4 a, uint4 b);
template <> __device__ __forceinline__ void mma16<bf16_t>(f32x16 &c, uint4 a, uint4 b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                0, 0, 0);
}
template <> __device__ __forceinline__ void mma16<f16_t>(f32x16 &c, uint4 a, uint4 b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                               0, 0);
}
// uint8 runs through the signed instruction: every operand is congruent to its signed
// reinterpretation modulo 2^8, so the wrapped sums agree modulo 2^32 and the truncated
// 8-bit results are identical.
template <> __device__ __forceinline__ void mma16<int8_t>(i32x16 &c, uint4 a, uint4 b) {
    c = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0,
                                              0, 0);
}
template <> __device__ __forceinline__ void mma16<uint8_t>(i32x16 &c, uint4 a, uint4 b) { mma16<int8_t>(c, a, b); }

// 16 x 16 x 32 blocks (16-bit inputs only).  Per flop they draw markedly less power than the
// 32 x 32 x 16 form: a probe that streams register-resident N(0,1) bf16 operands through each
// shape runs the 16 x 16 x 32 one at ~2.0 GHz and the 32 x 32 x 16 one at ~1.7 GHz under the
// board's power limit, and the large GEMMs are power limited.  Lane l holds index l % 16 and
// 8 consecutive k at 8 (l / 16) of both operands; the result block gives lane l rows
// 4 (l / 16) .. +3 of column l % 16.
typedef float f32x4 __attribute__((ext_vector_type(4)));
template <class T, int MS> struct AccT { using type = typename AccV<T>::type; };
template <class T> struct AccT<T, 16> { using type = f32x4; };
template <> struct AccT<int8_t, 16> { using type = i32x4; };
template <> struct AccT<uint8_t, 16> { using type = i32x4; };
template <class T> __device__ __forceinline__ void mma16x16(typename AccT<T, 16>::type &c, uint4 a, uint4 b);
template <> __device__ __forceinline__ void mma16x16<bf16_t>(f32x4 &c, uint4 a, uint4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                0);
}
template <> __device__ __forceinline__ void mma16x16<f16_t>(f32x4 &c, uint4 a, uint4 b) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}
// 8-bit: 16 x 16 x 64, 16 consecutive k per lane (k group l / 16); uint8 runs on the signed form
// like the 32 x 32 blocks (the products agree modulo 2^8, the width of the uint8 output)
template <> __device__ __forceinline__ void mma16x16<int8_t>(i32x4 &c, uint4 a, uint4 b) {
    c = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, a), __builtin_bit_cast(i32x4, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ void mma16x16<uint8_t>(i32x4 &c, uint4 a, uint4 b) { mma16x16<int8_t>(c, a, b); }
template <class T, int MS> __device__ __forceinline__ void mma_blk(typename AccT<T, MS>::type &c, uint4 a, uint4 b) {
    if constexpr (MS == 16)
        mma16x16<T>(c, a, b);
    else
        mma16<T>(c, a, b);
}

__device__ __forceinline__ int swz_k(int row) { return (row & 7) ^ ((row >> 3) & 3); }
// The same for K-major tiles read as 16 x 16 fragments (16 rows x one 16-byte chunk per k group
// per ds_read_b128): `row & 7` is conflict-free for that pattern (4 LDS cycles per read on
// MI355X, against 8 with `swz_k`, whose row-bit-3 term collides there).
__device__ __forceinline__ int swz_k16(int row) { return row & 7; }
// Chunk swizzle of M/N-major rows.  16-bit: {0, 4, 10, 14}[k & 3]; 8-bit: 2 (k & 7), which
// puts the 8 k-rows x 2 chunks that a 32-lane slice of one ds_read_b64_tr_b8 touches on 16
// distinct 16-byte bank groups (for 256-byte rows).  Limited to the chunks of one row.
// 16-bit 128-byte rows (CPR 8): a 32-lane slice of one ds_read_b64_tr_b16 reads 4 chunks of
// k-rows k0 .. k0 + 3; rows k and k + 1 already sit in opposite halves of the 64 banks, so the
// swizzle 4 ((k >> 1) & 1) puts k and k + 2 on opposite halves of the row (all 64 banks once);
// {0, 4, 10, 14} & 7 put them on the same 4 chunks, two LDS cycles per slice instead of one.
template <int CPR, int ES> __device__ __forceinline__ int swz_mn(int k) {
    if constexpr (ES == 2 && CPR == 8) {
        return 4 * ((k >> 1) & 1);
    } else if constexpr (ES == 2) {
        const int f = ((k & 1) << 2) | ((k & 2) ? 10 : 0);
        return f & (CPR - 1);
    } else {
        return (2 * (k & 7)) & (CPR - 1);
    }
}
// The same for the 16 x 16 x 32 fragments of 16-bit M/N-major rows: a 32-lane slice of one
// ds_read_b64_tr_b16 reads k-rows k0 + {0..3} and k0 + 8 + {0..3} of the same 16 columns (two
// chunks), so the swizzle 4 (k & 3) + 2 ((k >> 3) & 1) spreads those 8 rows x 2 chunks over 16
// distinct 16-byte bank groups.  It ignores k bits 2 and 5, which the per-read offsets add.
template <int CPR> __device__ __forceinline__ int swz_mn16(int k) {
    static_assert(CPR >= 16, "rows of at least 256 bytes");
    return 4 * (k & 3) + 2 * ((k >> 3) & 1);
}
// 8-bit rows read as 16 x 16 x 64 fragments: a 32-lane slice of one ds_read_b64_tr_b8 reads
// k-rows k0 + {0..7} and k0 + 16 + {0..7} of one 16-column chunk, which 2 (k & 7) + (k >> 4) & 1
// puts on 16 distinct 16-byte bank groups.
template <int CPR> __device__ __forceinline__ int swz_mn16_b8(int k) {
    static_assert(CPR >= 16, "rows of at least 256 bytes");
    return 2 * (k & 7) + ((k >> 4) & 1);
}

__device__ __forceinline__ MB_LDS char *lds_ptr(const char *p) { return (MB_LDS char *)(MB_LDS void *)p; }
__device__ __forceinline__ uint32_t lds_addr(const char *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_ptr(p));
}

// One operand tile: ROWS (M or N) x 128 bytes of K (64 16-bit or 128 8-bit elements), read as
// fragments of MS x MS MFMA blocks (MS = 32: 32 x 32 x 16 / 32 x 32 x 32; MS = 16: 16 x 16 x 32).
template <int ROWS, int NW, bool KC, int ES = 2, int MS = 32> struct Tile16 {
    static constexpr int BYTES = ROWS * 128;
    static constexpr int SEGS = BYTES / 1024;      // 1 KiB direct-load segments
    static constexpr int PER_WAVE = (SEGS + NW - 1) / NW;
    static constexpr int RB = ROWS * ES;           // MN-major row bytes
    static constexpr int CPR = RB / 16;            // MN-major chunks per row
    static constexpr int EPC = 16 / ES;            // elements per 16-byte chunk
    static_assert(ROWS % 32 == 0 && (KC || RB >= (ES == 2 ? 128 : 64)), "tile rows");
    static_assert(MS == 32 || MS == 16, "32 x 32 or 16 x 16 blocks");
    // chunk swizzle of K-major rows
    __device__ __forceinline__ static int swzk(int row) {
        if constexpr (MS == 16)
            return swz_k16(row);
        else
            return swz_k(row);
    }
    __device__ __forceinline__ static int swz(int k) {
        if constexpr (MS == 16 && ES == 2)
            return swz_mn16<CPR>(k);
        else if constexpr (MS == 16)
            return swz_mn16_b8<CPR>(k);
        else
            return swz_mn<CPR, ES>(k);
    }

    // Byte offset (relative to the resource base = element (row0, k0)) of the chunk a lane
    // loads for segment `seg`, or kOOB.
    __device__ __forceinline__ static uint32_t src_offset(int seg, int lane, int64_t ld, int rows_left,
                                                          int k_left) {
        const int byte = seg * 1024 + lane * 16;
        if constexpr (KC) {
            const int r = byte >> 7, p = (byte >> 4) & 7;
            const int c = p ^ swzk(r);
            if (r >= rows_left || c * EPC >= k_left) return kOOB;
            return (uint32_t)(((int64_t)r * ld + c * EPC) * ES);
        } else {
            const int k = byte / RB, p = (byte % RB) >> 4;
            const int c = p ^ swz(k);
            if (k >= k_left || c * EPC >= rows_left) return kOOB;
            return (uint32_t)(((int64_t)k * ld + c * EPC) * ES);
        }
    }

    // Lane-dependent LDS byte offset of the fragment of MFMA block `j` (32 rows) at k-step 0;
    // k-steps and blocks j' = j (mod 2 for KC) add compile-time constants.
    //   16-bit transposing read: a 16-lane group reads 4 k-rows x 16 columns (lane L gives 4
    //   columns of k-row L / 4) and returns column L's 4 k values to lane L.
    //   8-bit transposing read: a 16-lane group reads 8 k-rows x 16 columns (lane L gives 8
    //   columns of k-row L / 2) and returns column L's 8 k values to lane L.
    __device__ __forceinline__ static int frag_base(int row0, int lane, int j) {
        if constexpr (KC) {
            const int row = row0 + (lane & 31);
            return row * 128;   // chunk part is added per step (swizzle depends on lane only)
        } else if constexpr (ES == 2) {
            const int kr = (lane & 15) >> 2;   // k row within the 4-row group
            const int col = row0 + 32 * j + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
            return (kr + 8 * (lane >> 5)) * RB + (((col >> 3) ^ swz_mn<CPR, ES>(kr)) << 4) + ((col & 7) << 1);
        } else {
            const int kr = (lane & 15) >> 1;   // k row within the 8-row group
            const int col = row0 + 32 * j + 16 * ((lane >> 4) & 1) + 8 * (lane & 1);
            return (kr + 16 * (lane >> 5)) * RB + (((col >> 4) ^ swz_mn<CPR, ES>(kr)) << 4) + (col & 15);
        }
    }

    // 16 x 16 fragments: lane l reads index l % 16 of block j (16 rows) and 16 bytes of k for
    // k group l / 16: 16-bit (16 x 16 x 32) the 8 k at 32 s + 8 (l / 16), 8-bit (16 x 16 x 64)
    // the 16 k at 64 s + 16 (l / 16).  K-major: one 16-byte chunk; M/N-major: two transposing
    // reads, of 4 k (16-bit: k-row 8 (l / 16) + (l % 16) / 4 + 4 t of columns 4 (l % 4) .. +3)
    // or of 8 k (8-bit: k-row 16 (l / 16) + (l % 16) / 2 + 8 t of columns 8 (l % 2) .. +7).
    __device__ __forceinline__ static int frag_base16(int row0, int lane, int j) {
        if constexpr (KC) {
            return (row0 + (lane & 15)) * 128;   // row0 is a multiple of 32
        } else if constexpr (ES == 2) {
            const int k = 8 * (lane >> 4) + ((lane & 15) >> 2);
            const int col = row0 + 16 * j + 4 * (lane & 3);
            return k * RB + (((col >> 3) ^ swz(k)) << 4) + ((col & 7) << 1);
        } else {
            const int k = 16 * (lane >> 4) + ((lane & 15) >> 1);
            const int col = row0 + 16 * j + 8 * (lane & 1);
            return k * RB + (((col >> 4) ^ swz(k)) << 4) + (col & 15);
        }
    }
    __device__ __forceinline__ static uint4 frag16(const char *lds, int base, int lane, int s, int j) {
        if constexpr (KC) {
            const int row = 16 * (j & 1) + (lane & 15);   // the swizzle is periodic in 32 rows
            const int chunk = (4 * s + (lane >> 4)) ^ swzk(row);
            return *(const uint4 *)(lds + base + j * 16 * 128 + (chunk << 4));
        } else {
            uint4 out;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                uint2 u;
                if constexpr (ES == 2) {
                    const int koff = (32 * s + 4 * t) * RB;
                    bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MB_LDS bf16x4 *)(lds_ptr(lds) + base + koff));
                    u = __builtin_bit_cast(uint2, v);
                } else {
                    const int koff = (64 * s + 8 * t) * RB;
                    i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MB_LDS i32x2 *)(lds_ptr(lds) + base + koff));
                    u = __builtin_bit_cast(uint2, v);
                }
                if (t == 0) {
                    out.x = u.x;
                    out.y = u.y;
                } else {
                    out.z = u.x;
                    out.w = u.y;
                }
            }
            return out;
        }
    }

    __device__ __forceinline__ static uint4 frag(const char *lds, int base, int lane, int s, int j) {
        if constexpr (KC) {
            const int row = lane & 31;   // swizzle is periodic in 32 rows
            const int chunk = (2 * s + (lane >> 5)) ^ swz_k(row);
            return *(const uint4 *)(lds + base + j * 32 * 128 + (chunk << 4));
        } else {
            uint4 out;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                uint2 u;
                if constexpr (ES == 2) {
                    // k = 16 s + 8 (lane / 32) + 4 t + kr; the lane terms are folded into base
                    const int koff = (16 * s + 4 * t) * RB;
                    bf16x4 v =
                        __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MB_LDS bf16x4 *)(lds_ptr(lds) + base + koff));
                    u = __builtin_bit_cast(uint2, v);
                } else {
                    // k = 32 s + 16 (lane / 32) + 8 t + kr
                    const int koff = (32 * s + 8 * t) * RB;
                    i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((MB_LDS i32x2 *)(lds_ptr(lds) + base + koff));
                    u = __builtin_bit_cast(uint2, v);
                }
                if (t == 0) {
                    out.x = u.x;
                    out.y = u.y;
                } else {
                    out.z = u.x;
                    out.w = u.y;
                }
            }
            return out;
        }
    }
};

__device__ __forceinline__ void tile_coords16(int pid, int tiles_m, int tiles_n, int swz, int &tm, int &tn) {
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

// Store a wave's accumulators: acc[i][j] holds the MS x MS block at rows mw + MS j, columns
// nw + MS i; lane l owns row (l % MS) and columns 8 (r / 4) + 4 (l / MS) + r % 4 of register r
// (MS = 32: 16 registers; MS = 16: 4).
// Split-K slices write fp32 partial planes; otherwise the (optional) epilogue and one rounding.
template <class T, int TM, int TN, int MS = 32>
__device__ __forceinline__ void store_tile16(const GemmArgs &g, typename AccT<T, MS>::type (&acc)[TN][TM], int mw,
                                             int nw, int bz, int ks, int lane) {
    constexpr int NQ = MS * MS / 256;   // 4-register groups per lane
    using A = typename Tr<T>::acc;   // fp32, or the unsigned 32-bit wrapping accumulator
    // keep the store addressing from being hoisted above the main loop (where its 64-bit
    // addresses would be live across the loop and spill)
    asm volatile("" : "+s"(mw), "+s"(nw));
    const int mrow = lane % MS;
    const int nsub = 4 * (lane / MS);
    T *Cb = (T *)g.c + bz * g.c_bs;
    if (g.splits > 1 || g.planes) {
        A *ws = (A *)g.ws + ((int64_t)ks * g.batch + bz) * g.M * (int64_t)g.N;
        const bool vec = (g.N & 3) == 0;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int gm = mw + j * MS + mrow;
                if (gm >= g.M) continue;
                A *row = ws + (int64_t)gm * g.N;
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int gn = nw + i * MS + 8 * q + nsub;
                    if (vec && gn + 3 < g.N) {
                        A o[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[r] = (A)acc[i][j][4 * q + r];
                        uint4 u;
                        __builtin_memcpy(&u, o, 16);
                        *(uint4 *)(row + gn) = u;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (gn + r < g.N) row[gn + r] = (A)acc[i][j][4 * q + r];
                    }
                }
            }
    } else if (g.vec_ok && !g.epilogue) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int gm = mw + j * MS + mrow;
                if (gm >= g.M) continue;
                T *row = Cb + gm * g.c_rs;
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int gn = nw + i * MS + 8 * q + nsub;
                    if (gn + 3 < g.N) {
                        T o[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[r] = (T)acc[i][j][4 * q + r];
                        if constexpr (sizeof(T) == 2) {
                            uint2 u;
                            __builtin_memcpy(&u, o, 8);
                            *(uint2 *)(row + gn) = u;
                        } else {
                            uint32_t u;
                            __builtin_memcpy(&u, o, 4);
                            *(uint32_t *)(row + gn) = u;
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (gn + r < g.N) row[gn + r] = (T)acc[i][j][4 * q + r];
                    }
                }
            }
    } else if (g.vec_ok && g.bias_vec && !Tr<T>::is_complex) {
        // fused epilogue with 4-element vector bias loads and output stores (addmm's bias
        // row broadcast or a full bias matrix, both contiguous along N)
        const T *Bb = (const T *)g.bias + bz * g.bias_bs;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int gm = mw + j * MS + mrow;
                if (gm >= g.M) continue;
                T *row = Cb + gm * g.c_rs;
                const T *brow = Bb + gm * g.bias_rs;
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int gn = nw + i * MS + 8 * q + nsub;
                    if (gn + 3 < g.N) {
                        T bv[4], o[4];
                        if (g.beta_nz) __builtin_memcpy(bv, brow + gn, 4 * sizeof(T));
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            o[r] = Tr<T>::down(epi_apply<T>((A)acc[i][j][4 * q + r], bv + r, g.s, g.beta_nz, g.alpha_nz));
                        if constexpr (sizeof(T) == 2) {
                            uint2 u;
                            __builtin_memcpy(&u, o, 8);
                            *(uint2 *)(row + gn) = u;
                        } else {
                            uint32_t u;
                            __builtin_memcpy(&u, o, 4);
                            *(uint32_t *)(row + gn) = u;
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (gn + r < g.N)
                                store_out<T>(g, row + gn + r, (A)acc[i][j][4 * q + r],
                                             bz * g.bias_bs + gm * g.bias_rs + gn + r);
                    }
                }
            }
    } else {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const int gm = mw + j * MS + mrow;
                if (gm >= g.M) continue;
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int gn = nw + i * MS + 8 * q + nsub;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int n = gn + r;
                        if (n < g.N)
                            store_out<T>(g, Cb + gm * g.c_rs + n * g.c_cs, (A)acc[i][j][4 * q + r],
                                         bz * g.bias_bs + gm * g.bias_rs + n * g.bias_cs);
                    }
                }
            }
    }
}

// Output tile staged through LDS: the accumulators are converted and written into a BM x BN
// tile in LDS (row pitch padded by 16 bytes), then the workgroup stores whole rows with one
// 16-byte store per lane, consecutive lanes on consecutive chunks.  The direct stores of
// store_tile16 put 16-32 row fragments of 8-16 bytes in every store instruction, which holds
// products with a short K (where the output dominates the traffic) to about 2.5 TB/s of writes.
// Taken for row-major outputs with 16-byte aligned rows and no split-K planes; a fused epilogue
// is applied in registers before the tile is staged.
// Bank layout (64 banks of 4 bytes).  The 16 x 16 blocks (MS = 16) and 8-bit tiles write 16 rows
// per 16-lane group and use a 16-byte row pad.  The 32 x 32 blocks of 16-bit tiles write 32 rows
// of one 8-byte column piece per half-wave, which no 16-byte-granular pitch spreads over the
// banks, and the pad makes each 16-lane group of the row-wise reads straddle two rows' banks: their
// rows are unpadded, and the 8-byte pieces of row r sit at byte column c ^ xor_bytes(r), a
// permutation of the row's pieces (within each 256-byte window) that gives the 32 rows of a
// half-wave distinct banks (64-wide rows alternate bank halves, so row pairs share the XOR).
template <class T, int BM, int BN, int MS> struct CStage {
    static_assert(sizeof(T) <= 2, "the staged store packs 4 outputs into 8 or 4 bytes");
    static constexpr bool SWZ = sizeof(T) == 2 && MS == 32 && BN >= 64;
    static constexpr int PITCH = SWZ ? BN * 2 : BN * (int)sizeof(T) + 16;
    static constexpr int BYTES = BM * PITCH;
    __device__ __forceinline__ static int xor_bytes(int row) {
        if constexpr (!SWZ)
            return 0;
        else if constexpr (BN == 64)
            return 8 * ((row >> 1) & 15);
        else
            return 8 * (row & 31);
    }
};

template <class T> __device__ __forceinline__ bool staged_store_ok(const GemmArgs &g) {
    return g.splits <= 1 && !g.planes && g.c_cs == 1 && ((g.c_rs * (int64_t)sizeof(T)) & 15) == 0 &&
           (g.batch == 1 || ((g.c_bs * (int64_t)sizeof(T)) & 15) == 0) && (((uintptr_t)g.c) & 15) == 0;
}

// this wave's accumulators (the block layout of store_tile16) into the staged tile; mw / nw are
// tile-relative and m0 / n0 the tile's origin in C.  A fused epilogue (alpha, beta and the bias
// read at the output's coordinates) is applied before the one rounding, as store_tile16 does.
template <class T, int TM, int TN, int MS, class CS>
__device__ __forceinline__ void stage_acc(const GemmArgs &g, char *ct, typename AccT<T, MS>::type (&acc)[TN][TM],
                                          int mw, int nw, int m0, int n0, int bz, int lane) {
    constexpr int NQ = MS * MS / 256;
    using A = typename Tr<T>::acc;
    const int mrow = lane % MS, nsub = 4 * (lane / MS);
    // keep the bias addressing from being hoisted above the main loop (its per-row offsets
    // would be live across the loop in scalar registers and spill)
    asm volatile("" : "+s"(mw), "+s"(nw), "+s"(m0), "+s"(n0), "+s"(bz));
    const T *Bb = (const T *)g.bias + bz * g.bias_bs;
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const int row = mw + j * MS + mrow, col = nw + i * MS + 8 * q + nsub;
                T o[4];
                if (!g.epilogue) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) o[r] = (T)acc[i][j][4 * q + r];
                } else {
                    // bias elements past the edge of C are not read (their outputs are not stored)
                    const int gm = m0 + row, gn = n0 + col;
                    T bv[4] = {};
                    if (g.beta_nz && gm < g.M) {
                        const T *brow = Bb + gm * g.bias_rs;
                        if (g.bias_vec && gn + 3 < g.N) {
                            __builtin_memcpy(bv, brow + gn, 4 * sizeof(T));
                        } else {
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (gn + r < g.N) bv[r] = brow[(int64_t)(gn + r) * g.bias_cs];
                        }
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        o[r] = Tr<T>::down(epi_apply<T>((A)acc[i][j][4 * q + r], bv + r, g.s, g.beta_nz, g.alpha_nz));
                }
                char *dst = ct + row * CS::PITCH + ((col * (int)sizeof(T)) ^ CS::xor_bytes(row));
                if constexpr (sizeof(T) == 2) {
                    uint2 u;
                    __builtin_memcpy(&u, o, 8);
                    *(uint2 *)dst = u;
                } else {
                    uint32_t u;
                    __builtin_memcpy(&u, o, 4);
                    *(uint32_t *)dst = u;
                }
            }
}

// element k of a 16-byte chunk, picked from registers (a local array here would be placed in
// LDS by the compiler, 16 bytes per thread, and cost workgroups per CU)
template <class T> __device__ __forceinline__ T chunk_elem(const uint4 &v, int k) {
    constexpr int PER = 4 / (int)sizeof(T);
    const int w = k / PER;
    const uint32_t word = w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w;
    const uint32_t bits = word >> (8 * (int)sizeof(T) * (k % PER));
    if constexpr (sizeof(T) == 2)
        return __builtin_bit_cast(T, (uint16_t)bits);
    else
        return __builtin_bit_cast(T, (uint8_t)bits);
}

// the staged tile out to C rows m0.., columns n0.. (16 bytes per thread and step; the ragged
// right edge element by element); STREAM: non-temporal stores (an output larger than the cache)
template <class T, int BM, int BN, int MS, int NT, bool STREAM>
__device__ __forceinline__ void store_staged(const GemmArgs &g, const char *ct, int m0, int n0, int bz, int tid) {
    using CS = CStage<T, BM, BN, MS>;
    constexpr int EPC = 16 / (int)sizeof(T);
    constexpr int CPR = BN / EPC;
    T *Cb = (T *)g.c + bz * g.c_bs;
    const int rows = min(BM, g.M - m0), cols = min(BN, g.N - n0);
    for (int c = tid; c < rows * CPR; c += NT) {
        const int r = c / CPR, col = (c % CPR) * EPC;
        if (col >= cols) continue;
        const int x = CS::xor_bytes(r);   // 16-byte chunk col, its 8-byte halves swapped when x & 8
        uint4 v = *(const uint4 *)(ct + r * CS::PITCH + (((col * (int)sizeof(T)) ^ x) & ~15));
        if (x & 8) v = make_uint4(v.z, v.w, v.x, v.y);
        T *dst = Cb + (int64_t)(m0 + r) * g.c_rs + n0 + col;
        if (col + EPC <= cols) {
            if constexpr (STREAM) {
                typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
                __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, (u32x4_t *)dst);
            } else {
                *(uint4 *)dst = v;
            }
        } else {
            for (int k = 0; k < cols - col; ++k) dst[k] = chunk_elem<T>(v, k);
        }
    }
}

// KTAIL: some K slice ends inside a stage (its last stage is zero-filled past the
// edge).  Without it the main loop carries no edge logic.
template <class T, int BM, int BN, int WM, int WN, bool A_KC, bool B_KC, bool KTAIL>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm16(GemmArgs g) {
    constexpr int NW = WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int ES = sizeof(T);
    constexpr int BK = 128 / ES;   // elements of K per stage
    using TA = Tile16<BM, NW, A_KC, ES>;
    using TB = Tile16<BN, NW, B_KC, ES>;
    constexpr int STAGE = TA::BYTES + TB::BYTES;
    static_assert(TM >= 1 && TN >= 1, "wave tile");
    // LDS read instructions per k-step (a transposing fragment takes two)
    constexpr int NREAD_RAW = TM * (A_KC ? 1 : 2) + TN * (B_KC ? 1 : 2);
    constexpr int NREAD = NREAD_RAW < TM * TN ? NREAD_RAW : TM * TN;
    using CS = CStage<T, BM, BN, 32>;
    constexpr int SMEM = 2 * STAGE > CS::BYTES ? 2 * STAGE : CS::BYTES;

    __shared__ __attribute__((aligned(1024))) char smem[SMEM];
    __shared__ __attribute__((aligned(256))) char pf_junk[256];
    const uint32_t smem_lds = lds_addr(smem);   // LDS byte address of smem
    const uint32_t junk_lds = lds_addr(pf_junk);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int tiles_m = cdiv(g.M, BM), tiles_n = cdiv(g.N, BN);
    int tm, tn;
    tile_coords16(blockIdx.x, tiles_m, tiles_n, g.swz, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);
    const int klen = kend - kbeg;
    const int nk = cdiv(klen, BK);
    const int nfull = klen / BK;   // stages without a K edge
    const int64_t lda = A_KC ? g.a_rs : g.a_cs;
    const int64_t ldb = B_KC ? g.b_cs : g.b_rs;
    const int rows_a = g.M - m0, rows_b = g.N - n0;
    const int stepa = (int)((A_KC ? (int64_t)BK : (int64_t)BK * lda) * ES);
    const int stepb = (int)((B_KC ? (int64_t)BK : (int64_t)BK * ldb) * ES);
    // this lane's L2 prefetch line (full stages; the K-edge stage recomputes it)
    const uint32_t pfoff = pf_assign<BM, BN, A_KC, B_KC, ES>(wave, lane, tm, tn, lda, ldb, rows_a, rows_b, BK);
    const bool pf_on_a = wave == 0;

    // loop-invariant per-lane source offsets (full stages)
    uint32_t offa[TA::PER_WAVE], offb[TB::PER_WAVE];
#pragma unroll
    for (int i = 0; i < TA::PER_WAVE; ++i) {
        const int seg = wave + i * NW;
        offa[i] = seg < TA::SEGS ? TA::src_offset(seg, lane, lda, rows_a, BK) : kOOB;
    }
#pragma unroll
    for (int i = 0; i < TB::PER_WAVE; ++i) {
        const int seg = wave + i * NW;
        offb[i] = seg < TB::SEGS ? TB::src_offset(seg, lane, ldb, rows_b, BK) : kOOB;
    }
    // lane-dependent LDS fragment offsets
    int fba[A_KC ? 1 : TM], fbb[B_KC ? 1 : TN];
#pragma unroll
    for (int j = 0; j < (A_KC ? 1 : TM); ++j) fba[j] = TA::frag_base(wm * WTM, lane, j);
#pragma unroll
    for (int j = 0; j < (B_KC ? 1 : TN); ++j) fbb[j] = TB::frag_base(wn * WTN, lane, j);

    // Chained batch entries: a short K slice (at most four stages) over more batch entries than
    // the grid has z-blocks.  Each workgroup runs the stages of its entries as one stream
    // through the two LDS buffers: the loads of the stream's next stage, which is the next
    // entry's first stage after an entry's last, are issued before the current stage's
    // MFMAs, so the next entry's load latency overlaps this entry's last stage and epilogue
    // instead of following them (short-K batched products, e.g. attention scores with a
    // head dimension of 64).  The output is staged in the buffer of the entry's last stage,
    // which needs the staged tile to fit one stage (compiled for 16-bit tiles of at most
    // 128 x 128: in the 8-bit tiles the second loop cost a wave per SIMD of occupancy).
    constexpr bool CHAIN = ES == 2 && CS::BYTES <= STAGE && BM * BN <= 128 * 128;   // tiles that may chain
    if (CHAIN && nk >= 1 && nk <= 4 && (int)gridDim.z < g.batch) {
        // stage kt of batch entry e into buffer buf
        auto load_es = [&](int e, int kt, int buf) {
            const T *Ae = (const T *)g.a + e * g.a_bs + (A_KC ? (int64_t)m0 * lda + kbeg : (int64_t)kbeg * lda + m0);
            const T *Be = (const T *)g.b + e * g.b_bs + (B_KC ? (int64_t)n0 * ldb + kbeg : (int64_t)kbeg * ldb + n0);
            const i32x4 rae = make_rsrc(Ae), rbe = make_rsrc(Be);
            const uint32_t base = smem_lds + buf * STAGE;
            const bool full = !KTAIL || kt < nfull;
            const int kleft = klen - kt * BK;
#pragma unroll
            for (int i = 0; i < TA::PER_WAVE; ++i) {
                const int seg = wave + i * NW;
                if (TA::SEGS % NW == 0 || seg < TA::SEGS)
                    dma16(rae, base + seg * 1024, full ? offa[i] : TA::src_offset(seg, lane, lda, rows_a, kleft),
                          kt * stepa);
            }
#pragma unroll
            for (int i = 0; i < TB::PER_WAVE; ++i) {
                const int seg = wave + i * NW;
                if (TB::SEGS % NW == 0 || seg < TB::SEGS)
                    dma16(rbe, base + TA::BYTES + seg * 1024, full ? offb[i] : TB::src_offset(seg, lane, ldb, rows_b, kleft),
                          kt * stepb);
            }
        };
        typename AccV<T>::type acc[TN][TM];
        auto zero_acc = [&]() {
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
        };
        uint4 fa[2][TM], fb[2][TN];
        auto read_frags = [&](const char *cur, int s, int slot) {
#pragma unroll
            for (int j = 0; j < TM; ++j) fa[slot][j] = TA::frag(cur, fba[A_KC ? 0 : j], lane, s, A_KC ? j : 0);
#pragma unroll
            for (int i = 0; i < TN; ++i) fb[slot][i] = TB::frag(cur + TA::BYTES, fbb[B_KC ? 0 : i], lane, s, B_KC ? i : 0);
        };
        auto mma_step = [&](int slot) {
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j) mma16<T>(acc[i][j], fb[slot][i], fa[slot][j]);
        };
        zero_acc();
        int e = blockIdx.z, kt = 0, buf = 0;
        load_es(e, 0, 0);
        while (true) {
            vm_wait_all();     // this wave's loads of stage (e, kt), and earlier stores
            __syncthreads();   // stage (e, kt) landed everywhere; the other buffer is read out
            const bool last = kt + 1 == nk;
            const int ne = last ? e + (int)gridDim.z : e, nkt = last ? 0 : kt + 1;
            if (ne < g.batch) load_es(ne, nkt, buf ^ 1);
            char *cur = smem + buf * STAGE;
            read_frags(cur, 0, 0);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if (s < 3) read_frags(cur, s + 1, (s + 1) & 1);
                mma_step(s & 1);
            }
            if (last) {
                __syncthreads();   // every wave is done with this stage before it holds the output
                if (staged_store_ok<T>(g)) {
                    stage_acc<T, TM, TN, 32, CS>(g, cur, acc, wm * WTM, wn * WTN, m0, n0, e, lane);
                    __syncthreads();
                    if (g.c_stream)
                        store_staged<T, BM, BN, 32, 64 * NW, true>(g, cur, m0, n0, e, tid);
                    else
                        store_staged<T, BM, BN, 32, 64 * NW, false>(g, cur, m0, n0, e, tid);
                } else {
                    store_tile16<T, TM, TN>(g, acc, m0 + wm * WTM, n0 + wn * WTN, e, ks, lane);
                }
                zero_acc();
                if (ne >= g.batch) break;
            }
            e = ne;
            kt = nkt;
            buf ^= 1;
        }
        return;
    }

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        // resource bases: element (row0, kbeg) of each operand tile
        const T *Ab = (const T *)g.a + bz * g.a_bs + (A_KC ? (int64_t)m0 * lda + kbeg : (int64_t)kbeg * lda + m0);
        const T *Bb = (const T *)g.b + bz * g.b_bs + (B_KC ? (int64_t)n0 * ldb + kbeg : (int64_t)kbeg * ldb + n0);
        const i32x4 ra = make_rsrc(Ab), rb = make_rsrc(Bb);

        auto load_stage = [&](int kt, int buf) {
            const uint32_t base = smem_lds + buf * STAGE;
            if (!KTAIL || kt < nfull) {
#pragma unroll
                for (int i = 0; i < TA::PER_WAVE; ++i) {
                    const int seg = wave + i * NW;
                    if (TA::SEGS % NW == 0 || seg < TA::SEGS)
                        dma16(ra, base + seg * 1024, offa[i], kt * stepa);
                }
#pragma unroll
                for (int i = 0; i < TB::PER_WAVE; ++i) {
                    const int seg = wave + i * NW;
                    if (TB::SEGS % NW == 0 || seg < TB::SEGS)
                        dma16(rb, base + TA::BYTES + seg * 1024, offb[i], kt * stepb);
                }
            } else {
                // the K edge: chunks past the slice end read as zeros
                const int kleft = klen - kt * BK;
#pragma unroll
                for (int i = 0; i < TA::PER_WAVE; ++i) {
                    const int seg = wave + i * NW;
                    if (TA::SEGS % NW == 0 || seg < TA::SEGS)
                        dma16(ra, base + seg * 1024, TA::src_offset(seg, lane, lda, rows_a, kleft),
                              kt * stepa);
                }
#pragma unroll
                for (int i = 0; i < TB::PER_WAVE; ++i) {
                    const int seg = wave + i * NW;
                    if (TB::SEGS % NW == 0 || seg < TB::SEGS)
                        dma16(rb, base + TA::BYTES + seg * 1024, TB::src_offset(seg, lane, ldb, rows_b, kleft),
                              kt * stepb);
                }
            }
            const int kp = kt + kPfDist;
            const uint32_t po = kp >= nk ? kOOB : (!KTAIL || kp < nfull) ? pfoff
                              : pf_assign<BM, BN, A_KC, B_KC, ES>(wave, lane, tm, tn, lda, ldb, rows_a, rows_b, klen - kp * BK);
            pf_line(pf_on_a ? ra : rb, junk_lds, po, kp * (pf_on_a ? stepa : stepb));
        };

        typename AccV<T>::type acc[TN][TM];
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

        uint4 fa[2][TM], fb[2][TN];
        auto read_frags = [&](const char *cur, int s, int slot) {
#pragma unroll
            for (int j = 0; j < TM; ++j) fa[slot][j] = TA::frag(cur, fba[A_KC ? 0 : j], lane, s, A_KC ? j : 0);
#pragma unroll
            for (int i = 0; i < TN; ++i) fb[slot][i] = TB::frag(cur + TA::BYTES, fbb[B_KC ? 0 : i], lane, s, B_KC ? i : 0);
        };
        auto mma_step = [&](int slot) {
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j) mma16<T>(acc[i][j], fb[slot][i], fa[slot][j]);
        };

        if (nk > 0) {
            load_stage(0, 0);
            vm_wait_but_one();
            __syncthreads();
            read_frags(smem, 0, 0);
            if (nk > 1) load_stage(1, 1);
        }
        for (int kt = 0; kt < nk; ++kt) {
            const char *cur = smem + (kt & 1) * STAGE;
#pragma unroll
            for (int s = 0; s < 3; ++s) {
                read_frags(cur, s + 1, (s + 1) & 1);
                mma_step(s & 1);
                // one fragment read after each MFMA, so the reads of step s+1 spread over the
                // MFMAs of step s instead of stalling in a clump
#pragma unroll
                for (int r = 0; r < NREAD; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, TM * TN - NREAD, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (kt + 1 < nk) {
                vm_wait_but_one();   // this wave's loads of stage kt+1 have landed
                __syncthreads();   // stage kt+1 landed everywhere; stage kt fully read
                __builtin_amdgcn_sched_barrier(0);
                read_frags(smem + ((kt + 1) & 1) * STAGE, 0, 0);
                if (kt + 2 < nk) load_stage(kt + 2, kt & 1);
            }
            mma_step(1);
        }

        if (staged_store_ok<T>(g)) {
            __syncthreads();   // every wave is done with the operand stages
            stage_acc<T, TM, TN, 32, CS>(g, smem, acc, wm * WTM, wn * WTN, m0, n0, bz, lane);
            __syncthreads();
            if (g.c_stream)
                store_staged<T, BM, BN, 32, 64 * NW, true>(g, smem, m0, n0, bz, tid);
            else
                store_staged<T, BM, BN, 32, 64 * NW, false>(g, smem, m0, n0, bz, tid);
        } else {
            store_tile16<T, TM, TN>(g, acc, m0 + wm * WTM, n0 + wn * WTN, bz, ks, lane);
        }
        __syncthreads();   // LDS reuse by the next batch iteration
    }
}

// Thin products (a handful of vectors against a large matrix): the 32-wide operand tile is
// shared by every workgroup and stays in L2, the wide one is streamed from HBM exactly once.
// Instead of k_gemm16's two LDS buffers plus L2 prefetch (whose lines, at 64 workgroups per
// XCD, are evicted from the 4 MiB L2 before use), NST LDS buffers are in flight: the loads of
// stage kt + NST - 1 are issued right after the barrier that publishes stage kt, so each
// workgroup keeps (NST - 1) x 32 KiB of the wide operand on the way.  The matrix cores do
// 2 MFMAs per 16-deep k-step per wave; they are not the limit.
template <int N> __device__ __forceinline__ void vm_wait_n() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// Output tile and K slice of workgroup `pid` of a 1-D grid of n = tiles x splits workgroups:
// workgroup i runs on XCD i % 8, and the workgroups of one XCD take consecutive (slice, tile)
// indices, so the tiles of a K slice, which read the same slabs of A and B, share one XCD's L2
// (the remap is a bijection on [0, n) for any n).
__device__ __forceinline__ void slice_coords(int pid, int n, int tiles, int &tile, int &ks) {
    if (n >= 16) {
        const int xcd = pid & 7, idx = pid >> 3;
        const int base = n >> 3, rem = n & 7;
        pid = xcd * base + min(xcd, rem) + idx;
    }
    tile = pid % tiles;
    ks = pid / tiles;
}

// XMAP: one workgroup per (tile, K slice) on a 1-D grid in slice_coords order (deep-K products:
// few output tiles, many K slices); otherwise blockIdx.x is the tile and blockIdx.y the slice.
template <class T, int BM, int BN, int WM, int WN, bool A_KC, bool B_KC, bool KTAIL, int NST, bool XMAP = false,
          bool NTA = false, bool NTB = false>
__global__ __launch_bounds__(64 * WM * WN) void k_thin16(GemmArgs g) {
    constexpr int NW = WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int ES = sizeof(T);
    constexpr int BK = 128 / ES;
    using TA = Tile16<BM, NW, A_KC, ES>;
    using TB = Tile16<BN, NW, B_KC, ES>;
    constexpr int STAGE = TA::BYTES + TB::BYTES;
    static_assert(TM >= 1 && TN >= 1 && NST >= 3, "thin tile");
    static_assert(TA::SEGS % NW == 0 && TB::SEGS % NW == 0, "every wave issues the same loads");
    constexpr int LPS = TA::PER_WAVE + TB::PER_WAVE;   // LDS-direct loads per stage and wave
    static_assert((NST - 2) * LPS < 64, "vmcnt range");

    __shared__ __attribute__((aligned(1024))) char smem[NST * STAGE];
    const uint32_t smem_lds = lds_addr(smem);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int tiles_m = cdiv(g.M, BM), tiles_n = cdiv(g.N, BN);
    int tm, tn, ks;
    if constexpr (XMAP) {
        int tile;
        slice_coords(blockIdx.x, gridDim.x, tiles_m * tiles_n, tile, ks);
        tm = tile % tiles_m;
        tn = tile / tiles_m;
    } else {
        tile_coords16(blockIdx.x, tiles_m, tiles_n, g.swz, tm, tn);
        ks = blockIdx.y;
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);
    const int klen = kend - kbeg;
    const int nk = cdiv(klen, BK);
    const int nfull = klen / BK;
    const int64_t lda = A_KC ? g.a_rs : g.a_cs;
    const int64_t ldb = B_KC ? g.b_cs : g.b_rs;
    const int rows_a = g.M - m0, rows_b = g.N - n0;
    const int stepa = (int)((A_KC ? (int64_t)BK : (int64_t)BK * lda) * ES);
    const int stepb = (int)((B_KC ? (int64_t)BK : (int64_t)BK * ldb) * ES);

    uint32_t offa[TA::PER_WAVE], offb[TB::PER_WAVE];
#pragma unroll
    for (int i = 0; i < TA::PER_WAVE; ++i) offa[i] = TA::src_offset(wave + i * NW, lane, lda, rows_a, BK);
#pragma unroll
    for (int i = 0; i < TB::PER_WAVE; ++i) offb[i] = TB::src_offset(wave + i * NW, lane, ldb, rows_b, BK);
    int fba[A_KC ? 1 : TM], fbb[B_KC ? 1 : TN];
#pragma unroll
    for (int j = 0; j < (A_KC ? 1 : TM); ++j) fba[j] = TA::frag_base(wm * WTM, lane, j);
#pragma unroll
    for (int j = 0; j < (B_KC ? 1 : TN); ++j) fbb[j] = TB::frag_base(wn * WTN, lane, j);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const T *Ab = (const T *)g.a + bz * g.a_bs + (A_KC ? (int64_t)m0 * lda + kbeg : (int64_t)kbeg * lda + m0);
        const T *Bb = (const T *)g.b + bz * g.b_bs + (B_KC ? (int64_t)n0 * ldb + kbeg : (int64_t)kbeg * ldb + n0);
        const i32x4 ra = make_rsrc(Ab), rb = make_rsrc(Bb);

        auto load_stage = [&](int kt) {
            const uint32_t base = smem_lds + (kt % NST) * STAGE;
            if (!KTAIL || kt < nfull) {
#pragma unroll
                for (int i = 0; i < TA::PER_WAVE; ++i) dma16<NTA>(ra, base + (wave + i * NW) * 1024, offa[i], kt * stepa);
#pragma unroll
                for (int i = 0; i < TB::PER_WAVE; ++i)
                    dma16<NTB>(rb, base + TA::BYTES + (wave + i * NW) * 1024, offb[i], kt * stepb);
            } else {
                const int kleft = klen - kt * BK;
#pragma unroll
                for (int i = 0; i < TA::PER_WAVE; ++i)
                    dma16<NTA>(ra, base + (wave + i * NW) * 1024, TA::src_offset(wave + i * NW, lane, lda, rows_a, kleft),
                          kt * stepa);
#pragma unroll
                for (int i = 0; i < TB::PER_WAVE; ++i)
                    dma16<NTB>(rb, base + TA::BYTES + (wave + i * NW) * 1024,
                          TB::src_offset(wave + i * NW, lane, ldb, rows_b, kleft), kt * stepb);
            }
        };

        typename AccV<T>::type acc[TN][TM];
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

#pragma unroll
        for (int s = 0; s < NST - 1; ++s)
            if (s < nk) load_stage(s);
        for (int kt = 0; kt < nk; ++kt) {
            // stage kt has landed once at most the loads of stages kt+1 .. kt+NST-2 are pending
            if (kt + NST - 2 < nk) vm_wait_n<(NST - 2) * LPS>();
            else vm_wait_all();
            __syncthreads();   // stage kt visible to all waves; stage kt-1's buffer is free
            if (kt + NST - 1 < nk) load_stage(kt + NST - 1);
            const char *cur = smem + (kt % NST) * STAGE;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                uint4 fa[TM], fb[TN];
#pragma unroll
                for (int j = 0; j < TM; ++j) fa[j] = TA::frag(cur, fba[A_KC ? 0 : j], lane, s, A_KC ? j : 0);
#pragma unroll
                for (int i = 0; i < TN; ++i) fb[i] = TB::frag(cur + TA::BYTES, fbb[B_KC ? 0 : i], lane, s, B_KC ? i : 0);
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) mma16<T>(acc[i][j], fb[i], fa[j]);
            }
        }
        store_tile16<T, TM, TN>(g, acc, m0 + wm * WTM, n0 + wn * WTN, bz, ks, lane);
        __syncthreads();   // LDS reuse by the next batch iteration
    }
}

// The thin tiles 32 x 256 and 32 x 128: the vectors are the rows of A (K-contiguous), the
// matrix B is N-contiguous and streamed once with non-temporal loads (MI355X, 8 x 16384 @
// 16384^2 bf16, 4 K slices: 82.1 us against 88.1 us with cached loads).  4 buffers of 36 KiB
// (one workgroup per CU) or of 20 KiB (two).
template <class T, bool KTAIL>
hipError_t launch_thin16(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    if (!(t.bm == 32 && (t.bn == 256 || t.bn == 128) && t.wm == 1 && t.wn == 4 && a_kc && !b_kc))
        return hipErrorInvalidValue;
    if (t.bn == 256)
        hipLaunchKernelGGL((k_thin16<T, 32, 256, 1, 4, true, false, KTAIL, 4, false, false, true>), grid, dim3(256), 0, st, g);
    else
        hipLaunchKernelGGL((k_thin16<T, 32, 128, 1, 4, true, false, KTAIL, 4, false, false, true>), grid, dim3(256), 0, st, g);
    return hipGetLastError();
}

// The deep-K schedule (sched 2) of the 64 x 64 tile: products with few output tiles and a deep
// K, split into K slices so that ~256 workgroups stream the operands through a 4-deep ring of
// 16 KiB LDS-direct stages; the tiles of a slice run on one XCD (slice_coords), so each slab
// of A and B comes from HBM once.  Measured on MI355X for fp16 128 x 128 x 65536 (64 slices):
// 7.7 us against 11.6 us for the 2-D grid (tiles of a slice on different XCDs) and 14.4 us
// for the two-buffer 64 x 128 tile; deeper rings (5..8 stages) measured 8.5-9.4 us.
template <class T, bool A_KC, bool B_KC, bool KTAIL>
hipError_t launch_deepk16_t(const GemmArgs &g, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((k_thin16<T, 64, 64, 2, 2, A_KC, B_KC, KTAIL, 4, true>), grid, dim3(256), 0, st, g);
    return hipGetLastError();
}
template <class T, bool KTAIL>
hipError_t launch_deepk16(bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    if (a_kc) return b_kc ? launch_deepk16_t<T, true, true, KTAIL>(g, grid, st) : launch_deepk16_t<T, true, false, KTAIL>(g, grid, st);
    return b_kc ? launch_deepk16_t<T, false, true, KTAIL>(g, grid, st) : launch_deepk16_t<T, false, false, KTAIL>(g, grid, st);
}

// Ping-pong schedule of the 256 x 256 tile with 8 waves, two per SIMD (waves w and w + 4
// share SIMD w % 4).  The waves form two groups, 0..3 and 4..7, that alternate between a
// memory phase (all LDS fragment reads of one stage into registers, plus this wave's
// share of the LDS-direct prefetch) and a compute phase (the stage's 32 MFMAs back to back,
// every operand already in registers).  Group 1 runs one phase behind group 0, so on each
// SIMD one wave keeps the matrix core busy while the other feeds it; a workgroup barrier
// separates the phases:
//
//   phase      2k                    2k+1                  2k+2
//   group 0    read stage k,         compute stage k       read stage k+1,
//              prefetch stage k+1                          prefetch stage k+2
//   group 1    compute stage k-1,    read stage k          compute stage k,
//              prefetch stage k+1                          prefetch stage k+2
//
// Stage k lives in buffer k % 2 during phases 2k and 2k+1; its buffer is refilled (stage
// k+2) from phase 2k+2 on, after both groups read it.  Each wave waits for its own prefetch
// at the end of odd phases, before the barrier that publishes the stage.
//
// MS selects the MFMA block: 32 (32 x 32 x 16 / 32 x 32 x 32 int8, 4 k-steps per stage) or 16
// (16 x 16 x 32 / 16 x 16 x 64 int8, 2 k-steps).  The 16 x 16 form spends less power per flop,
// which is what bounds the large products, and runs without the L2 prefetch line: with the
// loads spread as here the prefetch only adds requests.
//
// BN = 128 (16 x 16 x 32 blocks only) halves the tile along N, for products with too few
// 256 x 256 tiles to fill the CUs: 128 x 32 wave tiles, 48 KiB stages.
template <class T, bool A_KC, bool B_KC, bool KTAIL, int MS = 32, int BN = 256>
__global__ __launch_bounds__(512) void k_gemm16pp(GemmArgs g) {
    static_assert(BN == 256 || (BN == 128 && MS == 16), "256 x 128 tiles use 16 x 16 x 32 blocks");
    constexpr int BM = 256, WM = 2, NW = 8;
    constexpr int WTM = 128, WTN = BN / 4, TM = WTM / MS, TN = WTN / MS;
    constexpr int ES = sizeof(T);
    constexpr int BK = 128 / ES, KSTEPS = MS == 16 ? 2 : 4;
    constexpr bool PF = MS == 32;
    using TA = Tile16<BM, NW, A_KC, ES, MS>;
    using TB = Tile16<BN, NW, B_KC, ES, MS>;
    constexpr int STAGE = TA::BYTES + TB::BYTES;
    using CS = CStage<T, BM, BN, MS>;
    constexpr int SMEM = 2 * STAGE > CS::BYTES ? 2 * STAGE : CS::BYTES;

    __shared__ __attribute__((aligned(1024))) char smem[SMEM];
    __shared__ __attribute__((aligned(256))) char pf_junk[256];
    const uint32_t smem_lds = lds_addr(smem);
    const uint32_t junk_lds = lds_addr(pf_junk);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int group = wave >> 2;
    const int wm = wave % WM, wn = wave / WM;
    const int tiles_m = cdiv(g.M, BM), tiles_n = cdiv(g.N, BN);
    int tm, tn;
    tile_coords16(blockIdx.x, tiles_m, tiles_n, g.swz, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int ks = blockIdx.y;
    const int kbeg = ks * g.k_chunk;
    const int kend = min(g.K, kbeg + g.k_chunk);
    const int klen = kend - kbeg;
    const int nk = cdiv(klen, BK);
    const int nfull = klen / BK;
    const int64_t lda = A_KC ? g.a_rs : g.a_cs;
    const int64_t ldb = B_KC ? g.b_cs : g.b_rs;
    const int rows_a = g.M - m0, rows_b = g.N - n0;
    const int stepa = (int)((A_KC ? (int64_t)BK : (int64_t)BK * lda) * ES);
    const int stepb = (int)((B_KC ? (int64_t)BK : (int64_t)BK * ldb) * ES);
    // this lane's L2 prefetch line (full stages; the K-edge stage recomputes it)
    const uint32_t pfoff = pf_assign<BM, BN, A_KC, B_KC, ES>(wave, lane, tm, tn, lda, ldb, rows_a, rows_b, BK);
    const bool pf_on_a = wave == 0;

    uint32_t offa[TA::PER_WAVE], offb[TB::PER_WAVE];
#pragma unroll
    for (int i = 0; i < TA::PER_WAVE; ++i) offa[i] = TA::src_offset(wave + i * NW, lane, lda, rows_a, BK);
#pragma unroll
    for (int i = 0; i < TB::PER_WAVE; ++i) offb[i] = TB::src_offset(wave + i * NW, lane, ldb, rows_b, BK);
    int fba[A_KC ? 1 : TM], fbb[B_KC ? 1 : TN];
#pragma unroll
    for (int j = 0; j < (A_KC ? 1 : TM); ++j)
        fba[j] = MS == 16 ? TA::frag_base16(wm * WTM, lane, j) : TA::frag_base(wm * WTM, lane, j);
#pragma unroll
    for (int j = 0; j < (B_KC ? 1 : TN); ++j)
        fbb[j] = MS == 16 ? TB::frag_base16(wn * WTN, lane, j) : TB::frag_base(wn * WTN, lane, j);

    for (int bz = blockIdx.z; bz < g.batch; bz += gridDim.z) {
        const T *Ab = (const T *)g.a + bz * g.a_bs + (A_KC ? (int64_t)m0 * lda + kbeg : (int64_t)kbeg * lda + m0);
        const T *Bb = (const T *)g.b + bz * g.b_bs + (B_KC ? (int64_t)n0 * ldb + kbeg : (int64_t)kbeg * ldb + n0);
        const i32x4 ra = make_rsrc(Ab), rb = make_rsrc(Bb);

        // this wave's share (1/8) of stage kt into buffer kt % 2
        auto prefetch = [&](int kt) {
            const uint32_t base = smem_lds + (kt & 1) * STAGE;
            if (!KTAIL || kt < nfull) {
#pragma unroll
                for (int i = 0; i < TA::PER_WAVE; ++i) dma16(ra, base + (wave + i * NW) * 1024, offa[i], kt * stepa);
#pragma unroll
                for (int i = 0; i < TB::PER_WAVE; ++i)
                    dma16(rb, base + TA::BYTES + (wave + i * NW) * 1024, offb[i], kt * stepb);
            } else {
                const int kleft = klen - kt * BK;
#pragma unroll
                for (int i = 0; i < TA::PER_WAVE; ++i)
                    dma16(ra, base + (wave + i * NW) * 1024, TA::src_offset(wave + i * NW, lane, lda, rows_a, kleft),
                          kt * stepa);
#pragma unroll
                for (int i = 0; i < TB::PER_WAVE; ++i)
                    dma16(rb, base + TA::BYTES + (wave + i * NW) * 1024,
                          TB::src_offset(wave + i * NW, lane, ldb, rows_b, kleft), kt * stepb);
            }
            if constexpr (PF) {
                const int kp = kt + kPfDist;
                const uint32_t po = kp >= nk ? kOOB : (!KTAIL || kp < nfull) ? pfoff
                                  : pf_assign<BM, BN, A_KC, B_KC, ES>(wave, lane, tm, tn, lda, ldb, rows_a, rows_b, klen - kp * BK);
                pf_line(pf_on_a ? ra : rb, junk_lds, po, kp * (pf_on_a ? stepa : stepb));
            }
        };
        // load `op` of prefetch(kt), in the same order: the A segments, the B segments, then the
        // L2-prefetch line (so the wait for "all but the most recent load" still works)
        constexpr int NOPS = TA::PER_WAVE + TB::PER_WAVE + (PF ? 1 : 0);
        // the wait for this wave's loads of a stage (the L2-prefetch line is left in flight)
        auto vm_wait_stage = [&]() {
            if constexpr (PF)
                vm_wait_but_one();
            else
                vm_wait_all();
        };
        // load `op` of prefetch(kt), in the same order: the A segments, the B segments, then the
        // L2-prefetch line.  EDGE: kt is the stage that holds the K edge (its offsets clip at the
        // slice end; computed here, so the full stages' code carries no select).
        auto prefetch_op = [&](auto edge_tag, int kt, int op) {
            constexpr bool EDGE = decltype(edge_tag)::value;
            const uint32_t base = smem_lds + (kt & 1) * STAGE;
            const int kleft = klen - kt * BK;
            if (op < TA::PER_WAVE) {
                const int seg = wave + op * NW;
                dma16(ra, base + seg * 1024, EDGE ? TA::src_offset(seg, lane, lda, rows_a, kleft) : offa[op], kt * stepa);
            } else if (op < TA::PER_WAVE + TB::PER_WAVE) {
                const int ib = op - TA::PER_WAVE, seg = wave + ib * NW;
                dma16(rb, base + TA::BYTES + seg * 1024, EDGE ? TB::src_offset(seg, lane, ldb, rows_b, kleft) : offb[ib],
                      kt * stepb);
            } else if constexpr (PF) {
                const int kp = kt + kPfDist;
                const uint32_t po = kp >= nk ? kOOB : (!KTAIL || kp < nfull) ? pfoff
                                  : pf_assign<BM, BN, A_KC, B_KC, ES>(wave, lane, tm, tn, lda, ldb, rows_a, rows_b, klen - kp * BK);
                pf_line(pf_on_a ? ra : rb, junk_lds, po, kp * (pf_on_a ? stepa : stepb));
            }
        };

        typename AccT<T, MS>::type acc[TN][TM];
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int r = 0; r < MS * MS / 64; ++r) acc[i][j][r] = 0;

        uint4 fa[KSTEPS][TM], fb[KSTEPS][TN];
        auto read_stage = [&](int kt) {
            const char *cur = smem + (kt & 1) * STAGE;
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    fa[s][j] = MS == 16 ? TA::frag16(cur, fba[A_KC ? 0 : j], lane, s, A_KC ? j : 0)
                                        : TA::frag(cur, fba[A_KC ? 0 : j], lane, s, A_KC ? j : 0);
#pragma unroll
                for (int i = 0; i < TN; ++i)
                    fb[s][i] = MS == 16 ? TB::frag16(cur + TA::BYTES, fbb[B_KC ? 0 : i], lane, s, B_KC ? i : 0)
                                        : TB::frag(cur + TA::BYTES, fbb[B_KC ? 0 : i], lane, s, B_KC ? i : 0);
            }
        };
        auto compute_stage = [&]() {
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) mma_blk<T, MS>(acc[i][j], fb[s][i], fa[s][j]);
            __builtin_amdgcn_s_setprio(0);
        };
        // the same MFMAs with prefetch(pk)'s loads issued one after each of the first NOPS
        // MFMAs (every second one for the half-length 16 x 16 MFMAs), so their issue (and the 5
        // wait states each carries) overlaps the matrix cores instead of delaying the first MFMA.
        // Unconditional: the iterations that prefetch run this body and the last two run
        // compute_stage.  A per-load condition (VALU compares feeding branches between the
        // MFMAs) stalled the MFMA stream: MI355X, bf16 8192^3, 1.45 M -> 1.28 M shader cycles
        // per call once the branches went (K-contiguous B: 1.54 M -> 1.38 M).
        constexpr int PF_EVERY = MS == 16 ? 2 : 1;
        auto compute_stage_pf = [&](auto edge_tag, int pk) {
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j) {
                        mma_blk<T, MS>(acc[i][j], fb[s][i], fa[s][j]);
                        const int idx = (s * TN + i) * TM + j;
                        if (idx % PF_EVERY == 0 && idx / PF_EVERY < NOPS) {
                            __builtin_amdgcn_sched_barrier(0);
                            prefetch_op(edge_tag, pk, idx / PF_EVERY);
                            __builtin_amdgcn_sched_barrier(0);
                        }
                    }
            __builtin_amdgcn_s_setprio(0);
        };
        auto phase_end = [&]() {
            __builtin_amdgcn_sched_barrier(0);
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
        };

        if (nk > 0) {
            prefetch(0);
            vm_wait_stage();
            phase_end();
            if (group == 0) {
                for (int kt = 0; kt < nk; ++kt) {
                    read_stage(kt);                 // phase 2kt
                    if (kt + 1 < nk) prefetch(kt + 1);
                    phase_end();
                    compute_stage();                // phase 2kt+1
                    vm_wait_stage();
                    phase_end();
                }
            } else {
                if (nk > 1) prefetch(1);            // phase 0
                phase_end();
                // iterations kt < pf_end prefetch stage kt+2 (phase 2kt+2); the first pf_full of
                // them prefetch a stage without a K edge
                // (uniform values: scalar loop tests, no VALU compare after the MFMAs)
                const int pf_end = __builtin_amdgcn_readfirstlane(nk - 2 > 0 ? nk - 2 : 0);
                const int pf_full = __builtin_amdgcn_readfirstlane(
                    KTAIL ? (nfull - 2 < pf_end ? (nfull - 2 > 0 ? nfull - 2 : 0) : pf_end) : pf_end);
                int kt = 0;
                for (; kt < pf_full; ++kt) {
                    read_stage(kt);                 // phase 2kt+1
                    vm_wait_stage();
                    phase_end();
                    compute_stage_pf(std::false_type{}, kt + 2);   // phase 2kt+2
                    phase_end();
                }
                if constexpr (KTAIL) {
                    for (; kt < pf_end; ++kt) {     // the stage with the K edge (at most one)
                        read_stage(kt);
                        vm_wait_stage();
                        phase_end();
                        compute_stage_pf(std::true_type{}, kt + 2);
                        phase_end();
                    }
                }
                for (; kt < nk; ++kt) {
                    read_stage(kt);
                    vm_wait_stage();
                    phase_end();
                    compute_stage();
                    if (kt + 1 < nk) phase_end();
                }
            }
        }
        if (staged_store_ok<T>(g)) {
            __syncthreads();   // both wave groups are done with the operand stages
            stage_acc<T, TM, TN, MS, CS>(g, smem, acc, wm * WTM, wn * WTN, m0, n0, bz, lane);
            __syncthreads();
            if (g.c_stream)
                store_staged<T, BM, BN, MS, 512, true>(g, smem, m0, n0, bz, tid);
            else
                store_staged<T, BM, BN, MS, 512, false>(g, smem, m0, n0, bz, tid);
        } else {
            store_tile16<T, TM, TN, MS>(g, acc, m0 + wm * WTM, n0 + wn * WTN, bz, ks, lane);
        }
        __syncthreads();   // LDS reuse by the next batch iteration
    }
}

// 16 x 16 blocks for every type: 16 x 16 x 32 for the 16-bit floats, 16 x 16 x 64 for 8-bit
// integers (MI355X, int8 4096^3, per layout: 67.0-69.8 us against 69.4-73.3 us with
// 32 x 32 x 32 blocks; bit-identical results)
template <class T, bool KTAIL, int BN = 256>
hipError_t launch16pp(bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    constexpr int MS = 16;
    dim3 block(512);
    if (a_kc && b_kc)
        hipLaunchKernelGGL((k_gemm16pp<T, true, true, KTAIL, MS, BN>), grid, block, 0, st, g);
    else if (a_kc && !b_kc)
        hipLaunchKernelGGL((k_gemm16pp<T, true, false, KTAIL, MS, BN>), grid, block, 0, st, g);
    else if (!a_kc && b_kc)
        hipLaunchKernelGGL((k_gemm16pp<T, false, true, KTAIL, MS, BN>), grid, block, 0, st, g);
    else
        hipLaunchKernelGGL((k_gemm16pp<T, false, false, KTAIL, MS, BN>), grid, block, 0, st, g);
    return hipGetLastError();
}

template <class T, int BM, int BN, int WM, int WN, bool KTAIL>
hipError_t launch16(bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    dim3 block(64 * WM * WN);
    if (a_kc && b_kc)
        hipLaunchKernelGGL((k_gemm16<T, BM, BN, WM, WN, true, true, KTAIL>), grid, block, 0, st, g);
    else if (a_kc && !b_kc)
        hipLaunchKernelGGL((k_gemm16<T, BM, BN, WM, WN, true, false, KTAIL>), grid, block, 0, st, g);
    else if (!a_kc && b_kc)
        hipLaunchKernelGGL((k_gemm16<T, BM, BN, WM, WN, false, true, KTAIL>), grid, block, 0, st, g);
    else
        hipLaunchKernelGGL((k_gemm16<T, BM, BN, WM, WN, false, false, KTAIL>), grid, block, 0, st, g);
    return hipGetLastError();
}

// Compiled 16-bit tiles: (BM, BN, WM, WN)
#define MB_M16_TILES(X) \
    X(256, 256, 2, 2)   \
    X(256, 256, 2, 4)   \
    X(256, 128, 2, 2)   \
    X(128, 256, 2, 2)   \
    X(128, 128, 2, 2)   \
    X(128, 64, 2, 2)    \
    X(64, 128, 2, 2)    \
    X(64, 64, 2, 2)

template <class T, bool KTAIL>
hipError_t launch16_typed(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
#define MB_M16_CASE(BM, BN, WM, WN) \
    if (t.bm == BM && t.bn == BN && t.wm == WM && t.wn == WN) \
        return launch16<T, BM, BN, WM, WN, KTAIL>(a_kc, b_kc, g, grid, st);
    MB_M16_TILES(MB_M16_CASE)
#undef MB_M16_CASE
    return hipErrorInvalidValue;
}

}  // namespace m16
}  // namespace mb
