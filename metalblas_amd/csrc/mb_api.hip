// C ABI and planner of libmetalblas_hip.so.
//
// The planner restates the decisions of the reference's L3 planners for gfx950
// (metalblas/float_dispatch.py:745-852 backend choice, :484-505 plan cache, :613-655 tile
// picker, :210-219 split-K regime; metalblas/integer_dispatch.py:92-117;
// metalblas/complex_dispatch.py:33-66 GEMV routing) and re-derives the numbers for 256 CUs
// and 160 KB of LDS: thin products (M or N <= 16) stream the matrix once through the GEMV
// families, aligned bf16/fp16/fp32/int8/uint8 products run on the matrix-core family, and
// everything else on the generic tiled kernel.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>
#include <string.h>

#include "../../include/metalblas_amd.h"
#include "launch.hpp"

using namespace mb;

// Scratch of the allocation-free entry point mb_gemm_noalloc (see scratch_address below).
static constexpr int64_t kScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

constexpr int64_t kI32Max = 2147483647;

struct Operand {
    const char *ptr;
    int64_t rs, cs, bs;
};

// Normalised problem (element strides, int64 sizes), possibly transposed.
struct Prob {
    int dt;
    int64_t batch, M, N, K;
    Operand a, b, c, bias;
    int conj_a, conj_b;
    int epilogue, beta_nz, alpha_nz;
    EpiScalars s;
    int backend;
    int32_t tile[8];
    int swz;
    int split_req;
    bool transposed;
    bool a_padded = false, b_padded = false;   // workspace copies, contiguous extent zero-padded
};

// A strided operand copied into the workspace in a layout the matrix-core loaders can stream
// (16-byte aligned base and leading dimension, the contiguous extent padded to a 16-byte
// multiple with zeros).
struct PackOp {
    bool on = false;
    int64_t off = 0;        // byte offset of the copy in the workspace
    PackArgs a{};           // source / destination strides and extents (dst pointer set at run)
};

struct Plan {
    int family = MB_FAMILY_NONE;
    Prob p;
    PackOp pack[2];           // A, B
    int64_t split_off = 0;    // workspace byte offset of the split-K partial planes
    // complex product run as the real product M x 2N x 2K (CplxExpandArgs)
    bool cplx = false;
    CplxExpandArgs cx{};      // B expansion (dst set at run time)
    int64_t cx_off = 0;
    bool cplx_reduce = false; // real GEMM writes fp32 planes; a complex reduction applies the
    GemmArgs cr{};            // epilogue and the output strides (ws set at run time)
    int cdt = 0;              // the complex dtype
    // GEMV
    GemvArgs gv{};
    bool gemv_dot = false;
    bool gemv_fast = false;   // streaming float kernels of gemv_fast.hip
    // MFMA / generic
    GemmArgs gg{};
    int gen_bt = 64;          // generic family: square output tile (64, 32 or 16)
    MfmaTile tile = {0, 0, 0, 0};
    bool a_kc = false, b_kc = false;
    int64_t ws_bytes = 0;
};

struct DevInfo {
    bool init = false;
    int cus = 256;
    int arch = 0;
    int64_t lds = 65536;
};
std::mutex g_dev_mu;
DevInfo g_dev[64];

const DevInfo &dev_info() {
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) d = 0;
    std::lock_guard<std::mutex> lk(g_dev_mu);
    DevInfo &di = g_dev[d];
    if (!di.init) {
        hipDeviceProp_t pr;
        if (hipGetDeviceProperties(&pr, d) == hipSuccess) {
            di.cus = pr.multiProcessorCount > 0 ? pr.multiProcessorCount : 256;
            di.lds = (int64_t)pr.sharedMemPerBlock;
            const char *n = pr.gcnArchName;
            if (strncmp(n, "gfx", 3) == 0) {
                int v = 0;
                for (const char *q = n + 3; *q >= '0' && *q <= '9'; ++q) v = v * 10 + (*q - '0');
                di.arch = v;
            }
        }
        di.init = true;
    }
    return di;
}

bool aligned(const void *p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }
int ilog2_floor(int64_t v) {
    int r = 0;
    while ((int64_t(1) << (r + 1)) <= v) ++r;
    return r;
}

// Internal descriptor flag (never accepted from a caller): the call runs on the static scratch
// of mb_gemm_noalloc, so a plan that needs more scratch than it holds is an error rather than a
// fall-back to the plan without scratch.
constexpr int32_t kFlagStaticScratch = 1 << 30;

// A caller's descriptor carrying an internal flag: the public entry points refuse it (only
// mb_gemm_noalloc sets kFlagStaticScratch, on its own copy of the descriptor).
bool internal_flags(const mb_gemm_desc *d) { return d && (d->flags & kFlagStaticScratch); }

int normalise(const mb_gemm_desc *d, Prob &p) {
    if (!d) return MB_ERR_INVALID_ARG;
    if (d->dtype < 0 || d->dtype >= MB_DTYPE_COUNT) return MB_ERR_UNSUPPORTED_DTYPE;
    if (d->backend < 0 || d->backend >= MB_BACKEND_COUNT) return MB_ERR_BAD_BACKEND;
    if (d->batch < 0 || d->M < 0 || d->N < 0 || d->K < 0) return MB_ERR_INVALID_ARG;
    if (d->batch > kI32Max || d->M > kI32Max || d->N > kI32Max || d->K > kI32Max) return MB_ERR_INVALID_ARG;
    if (d->flags & ~(MB_FLAG_DRY_RUN | kFlagStaticScratch)) return MB_ERR_INVALID_ARG;
    p.dt = d->dtype;
    p.batch = d->batch;
    p.M = d->M;
    p.N = d->N;
    p.K = d->K;
    p.a = {(const char *)d->a.ptr, d->a.row_stride, d->a.col_stride, d->a.batch_stride};
    p.b = {(const char *)d->b.ptr, d->b.row_stride, d->b.col_stride, d->b.batch_stride};
    p.c = {(const char *)d->c.ptr, d->c.row_stride, d->c.col_stride, d->c.batch_stride};
    p.bias = {(const char *)d->bias.ptr, d->bias.row_stride, d->bias.col_stride, d->bias.batch_stride};
    const bool cplx = p.dt == MB_DTYPE_C64 || p.dt == MB_DTYPE_C32;
    p.conj_a = cplx && d->conj_a;
    p.conj_b = cplx && d->conj_b;
    p.epilogue = d->epilogue != 0;
    p.beta_nz = p.epilogue && d->beta_nz;
    p.alpha_nz = p.epilogue ? (d->alpha_nz != 0) : 1;
    p.s.alpha_re = (float)d->alpha_re;
    p.s.alpha_im = (float)d->alpha_im;
    p.s.beta_re = (float)d->beta_re;
    p.s.beta_im = (float)d->beta_im;
    p.s.alpha_u = (uint64_t)d->alpha_int;
    p.s.beta_u = (uint64_t)d->beta_int;
    p.backend = d->backend;
    memcpy(p.tile, d->tile, sizeof(p.tile));
    p.swz = d->swizzle_log;
    p.split_req = d->split_k;
    p.transposed = false;
    if (p.batch == 0 || p.M == 0 || p.N == 0) return MB_OK;
    if (!p.c.ptr) return MB_ERR_INVALID_ARG;
    if (p.K > 0 && (!p.a.ptr || !p.b.ptr)) return MB_ERR_INVALID_ARG;
    if (p.beta_nz && !p.bias.ptr) return MB_ERR_INVALID_ARG;
    if (p.backend == MB_BACKEND_GEMV && p.M != 1 && p.N != 1) return MB_ERR_GEMV_SHAPE;
    return MB_OK;
}

// C^T = B^T A^T: swap operands and their row/col strides.
void transpose(Prob &p) {
    std::swap(p.M, p.N);
    Operand a = p.a, b = p.b;
    p.a = {b.ptr, b.cs, b.rs, b.bs};
    p.b = {a.ptr, a.cs, a.rs, a.bs};
    p.c = {p.c.ptr, p.c.cs, p.c.rs, p.c.bs};
    p.bias = {p.bias.ptr, p.bias.cs, p.bias.rs, p.bias.bs};
    std::swap(p.conj_a, p.conj_b);
    p.transposed = !p.transposed;
}

void fill_gemm_args(const Prob &p, GemmArgs &g) {
    memset(&g, 0, sizeof(g));
    g.a = p.a.ptr;
    g.b = p.b.ptr;
    g.c = (void *)p.c.ptr;
    g.bias = p.bias.ptr;
    g.a_rs = p.a.rs; g.a_cs = p.a.cs; g.a_bs = p.a.bs;
    g.b_rs = p.b.rs; g.b_cs = p.b.cs; g.b_bs = p.b.bs;
    g.c_rs = p.c.rs; g.c_cs = p.c.cs; g.c_bs = p.c.bs;
    g.bias_rs = p.bias.rs; g.bias_cs = p.bias.cs; g.bias_bs = p.bias.bs;
    g.M = (int)p.M; g.N = (int)p.N; g.K = (int)p.K; g.batch = (int)p.batch;
    g.conj_a = p.conj_a; g.conj_b = p.conj_b;
    g.epilogue = p.epilogue; g.beta_nz = p.beta_nz; g.alpha_nz = p.alpha_nz;
    // An output past the 256 MiB Infinity Cache is written with non-temporal stores (the
    // LDS-staged epilogue); smaller ones stay in the cache.  Measured on MI355X (bf16 bmm, us,
    // cached -> non-temporal): 48 x 2048 x 2048 x 64 (402 MB) 122 -> 103; 16 x 1024^3 (34 MB)
    // 41 -> 48, 96 x 512 x 512 x 64 (50 MB) 19 -> 27.
    g.c_stream = p.batch * p.M * p.N * dtype_size(p.dt) >= (int64_t(256) << 20);
    g.splits = 1;
    g.k_chunk = (int)(p.K > 0 ? p.K : 1);
    {
        const int es = dtype_size(p.dt);
        g.bias_vec = !p.beta_nz || (p.bias.cs == 1 && p.bias.rs % 4 == 0 && p.bias.bs % 4 == 0 &&
                                    aligned(p.bias.ptr, 4 * es));
    }
    g.swz = 0;
    g.s = p.s;
}

// ---- GEMV planning ----------------------------------------------------------------------
// Returns true and fills the plan when the thin side can be streamed by a GEMV family.
bool plan_gemv(const Prob &p, Plan &pl) {
    const int es = dtype_size(p.dt);
    const bool n_thin = p.N <= p.M;   // thin output dimension: N (matrix = A) or M (matrix = B)
    const int64_t nv = n_thin ? p.N : p.M;
    if (nv > 16) return false;
    GemvArgs g;
    memset(&g, 0, sizeof(g));
    bool dot;
    if (n_thin) {
        if (p.a.cs == 1) {
            dot = true;
            g.mat = p.a.ptr; g.mat_ld = p.a.rs;
        } else if (p.a.rs == 1) {
            dot = false;
            g.mat = p.a.ptr; g.mat_ld = p.a.cs;
        } else {
            return false;
        }
        g.mat_bs = p.a.bs;
        g.x = p.b.ptr; g.x_ks = p.b.rs; g.x_vs = p.b.cs; g.x_bs = p.b.bs;
        g.y = (void *)p.c.ptr; g.y_is = p.c.rs; g.y_vs = p.c.cs; g.y_bs = p.c.bs;
        g.bias = p.bias.ptr; g.bias_is = p.bias.rs; g.bias_vs = p.bias.cs; g.bias_bs = p.bias.bs;
        g.conj_mat = p.conj_a; g.conj_x = p.conj_b;
        g.rows = (int)p.M;
    } else {
        if (p.b.cs == 1) {
            dot = false;
            g.mat = p.b.ptr; g.mat_ld = p.b.rs;
        } else if (p.b.rs == 1) {
            dot = true;
            g.mat = p.b.ptr; g.mat_ld = p.b.cs;
        } else {
            return false;
        }
        g.mat_bs = p.b.bs;
        g.x = p.a.ptr; g.x_ks = p.a.cs; g.x_vs = p.a.rs; g.x_bs = p.a.bs;
        g.y = (void *)p.c.ptr; g.y_is = p.c.cs; g.y_vs = p.c.rs; g.y_bs = p.c.bs;
        g.bias = p.bias.ptr; g.bias_is = p.bias.cs; g.bias_vs = p.bias.rs; g.bias_bs = p.bias.bs;
        g.conj_mat = p.conj_b; g.conj_x = p.conj_a;
        g.rows = (int)p.N;
    }
    g.K = (int)p.K;
    g.nv = (int)nv;
    g.batch = (int)p.batch;
    g.epilogue = p.epilogue; g.beta_nz = p.beta_nz; g.alpha_nz = p.alpha_nz;
    g.s = p.s;
    g.splits = 1;
    g.k_chunk = g.K;
    g.grid_cap = 2 * dev_info().cus;
    const bool batched = p.batch > 1;
    bool fast = false;
    if (dot) {
        const int V = 16 / es;
        const bool mat_ok =
            aligned(g.mat, 16) && (g.mat_ld * es) % 16 == 0 && (!batched || (g.mat_bs * es) % 16 == 0) && (g.K % V) == 0;
        bool ok = mat_ok && g.x_ks == 1 && aligned(g.x, 16) && (!batched || (g.x_bs * es) % 16 == 0);
        ok = ok && (nv == 1 || (g.x_vs * es) % 16 == 0);
        g.vec_ok = ok;
        fast = ok && gemv_fast_dtype(p.dt);
        // complex64, one vector, no epilogue: the complex k_dot_wg stream (k_cdot_wg)
        if (p.dt == MB_DTYPE_C64 && ok && nv == 1 && !p.epilogue) fast = true;
        // X with its nv values contiguous per k (row-major thin X): exact power-of-two nv,
        // every k-row aligned to nv elements
        const int bucket = gemv_nv_bucket((int)nv);
        if (!fast && mat_ok && gemv_fast_dtype(p.dt) && nv > 1 && bucket == nv && g.x_vs == 1 &&
            g.x_ks % nv == 0 && aligned(g.x, (int)nv * es) && (!batched || g.x_bs % nv == 0)) {
            fast = true;
            g.x_row = 1;
        }
    } else {
        int V = gemv_axpy_vec(p.dt, (int)nv);
        if (gemv_fast_dtype(p.dt)) {
            const int Vf = gemv_fast_vec(p.dt);
            fast = aligned(g.mat, 16) && (g.mat_ld * es) % 16 == 0 && (!batched || (g.mat_bs * es) % 16 == 0) &&
                   (g.rows % Vf) == 0;
            if (fast) V = Vf;
        }
        const int vb = V * es;
        bool ok = aligned(g.mat, vb) && (g.mat_ld * es) % vb == 0 && (!batched || (g.mat_bs * es) % vb == 0);
        ok = ok && (g.rows % V) == 0;
        g.vec_ok = ok;
        const int vv = ok ? V : 1;
        const int64_t waves = ((int64_t)g.rows + 64 * vv - 1) / (64 * vv) * p.batch;
        const int cus = dev_info().cus;
        int64_t splits = (8LL * cus + waves - 1) / waves;   // about 8 waves per CU
        const int band = fast ? gemv_axpy_band_cols(p.dt, (int)nv, g.rows) : 0;
        int64_t max_splits = (p.K + 63) / 64;
        if (band > 0) {   // column-band kernel: one 4-wave workgroup per CU
            const int64_t blocks = ((int64_t)g.rows + band - 1) / band * p.batch;
            splits = (cus + blocks - 1) / blocks;
            // narrow matrices: slices of down to 32 rows, so the grid still covers the CUs
            if (blocks * max_splits < cus) max_splits = (p.K + 31) / 32;
        }
        if (splits > max_splits) splits = max_splits;
        if (splits > 256) splits = 256;
        if (splits < 1) splits = 1;
        if (splits > 1) {
            int64_t chunk = (p.K + splits - 1) / splits;
            chunk = (chunk + 7) / 8 * 8;
            splits = (p.K + chunk - 1) / chunk;
            g.k_chunk = (int)chunk;
            g.splits = (int)splits;
            pl.ws_bytes = splits * p.batch * nv * (int64_t)g.rows * acc_size(p.dt);
        }
    }
    pl.family = dot ? MB_FAMILY_GEMV_DOT : MB_FAMILY_GEMV_AXPY;
    pl.gemv_dot = dot;
    pl.gemv_fast = fast;
    pl.gv = g;
    return true;
}

// ---- matrix-core planning ---------------------------------------------------------------
// The compiled tile nearest to a requested one.  tile = (BM, BN, BK, WM, WN, schedule + 1):
// an explicit wave grid (WM, WN) and schedule are honoured when compiled; BK is fixed by the
// dtype.  The reference's (BM, BN, NSG) form for backend="mpp_tensor" leaves WM/WN at 0 and
// gets the default 2 x 2 wave grid.
// the thin-product tiles (k_thin_dot 64 x 16, k_thin_dot4 4 x 16, k_dotx 4 x 8, k_thin16 32 x 256
// and 32 x 128)
bool thin_tile(const MfmaTile &t) {
    return (t.bm == 64 && t.bn == 16) || (t.bm == 4 && t.bn == 16) || (t.bm == 4 && t.bn == 8) ||
           (t.bm == 32 && (t.bn == 256 || t.bn == 128));
}

// thin_ok: the thin-product tiles are candidates (only for plan_thin_mfma's own request)
MfmaTile snap_tile(int dt, const int32_t *t, bool a_kc, bool b_kc, bool thin_ok) {
    MfmaTile want = {t[0], t[1], 2, 2};
    if (t[3] > 0 && t[4] > 0) {
        want.wm = t[3];
        want.wn = t[4];
    }
    const int want_sched = t[5] > 0 ? t[5] - 1 : -1;
    MfmaTile list[32];
    const int n = mfma_list_tiles(dt, list, 32);
    int best = 0;
    double bestd = 1e30;
    for (int i = 0; i < n && i < 32; ++i) {
        // thin tiles: bf16 / fp16, 64 x 16 and 4 x 16 with both operands K-contiguous, 4 x 8
        // with A K-contiguous, 32 x 256 / 32 x 128 with A K-contiguous and B N-contiguous
        if (thin_tile(list[i]) &&
            (!thin_ok || (dt != MB_DTYPE_BF16 && dt != MB_DTYPE_F16) ||
             (list[i].bn == 16 ? !(a_kc && b_kc) : list[i].bn == 8 ? !a_kc : !(a_kc && !b_kc))))
            continue;
        double d = fabs(log2((double)list[i].bm / (want.bm > 0 ? want.bm : 1))) +
                   fabs(log2((double)list[i].bn / (want.bn > 0 ? want.bn : 1)));
        if (list[i].wm != want.wm || list[i].wn != want.wn) d += 0.01;
        if (want_sched >= 0 && list[i].sched != want_sched) d += 0.005;
        if (d < bestd) {
            bestd = d;
            best = i;
        }
    }
    return list[best];
}

// Orientation of an operand: 1 = contiguous along K, 0 = contiguous along M (A) / N (B),
// -1 = no unit stride.
int a_orient(const Prob &p) { return p.a.cs == 1 ? 1 : p.a.rs == 1 ? 0 : -1; }
int b_orient(const Prob &p) { return p.b.rs == 1 ? 1 : p.b.cs == 1 ? 0 : -1; }

// Can the matrix-core loaders stream this operand in place?  16-byte aligned base, leading
// dimension and batch stride, and the contiguous extent a multiple of 16 bytes (chunks never
// straddle the end of a row).  The LDS-direct loads would take misaligned rows too (their
// buffer loads accept any byte address), but misaligned they slowed the matrix-core kernels
// down by more than the operand copies cost, so such operands are copied.
bool operand_ok(const Operand &o, int orient, bool is_a, const Prob &p) {
    const int es = dtype_size(p.dt), E = 16 / es;
    if (orient < 0) return false;
    const bool kc = orient == 1;
    const int64_t ld = is_a ? (kc ? o.rs : o.cs) : (kc ? o.cs : o.rs);
    const int64_t contig = kc ? p.K : (is_a ? p.M : p.N);
    const bool padded = is_a ? p.a_padded : p.b_padded;   // the chunk past the end reads zeros
    if ((ld * es) % 16 || (!padded && contig % E)) return false;
    if (!aligned(o.ptr, 16) || (p.batch > 1 && (o.bs * es) % 16)) return false;
    return true;
}

bool mfma_layout_ok(const Prob &p, bool &a_kc, bool &b_kc) {
    if (!mfma_supported_dtype(p.dt)) return false;
    const int oa = a_orient(p), ob = b_orient(p);
    a_kc = oa == 1;
    b_kc = ob == 1;
    return operand_ok(p.a, oa, true, p) && operand_ok(p.b, ob, false, p);
}

// Plan workspace copies of the operands the loaders cannot stream in place (the reference's
// storage-offset views such as a 17-element offset, odd leading dimensions, K not a multiple
// of 16 bytes).  The copy keeps the operand's orientation (K-contiguous if it has no unit
// stride) and zero-pads the contiguous extent; when K is padded every K-contiguous operand
// is copied so that the padding contributes zeros.  Returns the workspace bytes used.
// Bit w of force_kc (0 = A, 1 = B) asks for that operand K-contiguous whatever its layout.
int64_t plan_packs(Prob &p, Plan &pl, int force_kc = 0) {
    const int es = dtype_size(p.dt), E = 16 / es;
    int64_t ws = 0;
    const char *placeholder = (const char *)(uintptr_t)4096;   // aligned stand-in until run time
    bool need[2];
    int orients[2];
    for (int which = 0; which < 2; ++which) {
        const bool is_a = which == 0;
        int orient = is_a ? a_orient(p) : b_orient(p);
        need[which] = !operand_ok(is_a ? p.a : p.b, orient, is_a, p);
        if (((force_kc >> which) & 1) && orient != 1) need[which] = true;
        if (orient < 0 || ((force_kc >> which) & 1)) orient = 1;
        if (orient == 1 && p.K % E) need[which] = true;
        orients[which] = orient;
    }
    // Both operands copied: zero-pad K to a whole stage (128 bytes of K) in both copies and run
    // the product over the padded K, so the matrix-core kernels need no K-edge handling (the
    // K-edge variants keep more registers live; 4097^3 bf16 spends 259 us in one).
    int64_t Kp = p.K;
    if (need[0] && need[1] && force_kc == 0) Kp = (p.K + 128 / es - 1) / (128 / es) * (128 / es);
    for (int which = 0; which < 2; ++which) {
        const bool is_a = which == 0;
        Operand &o = is_a ? p.a : p.b;
        const int orient = orients[which];
        if (!need[which]) continue;
        PackOp &pk = pl.pack[which];
        PackArgs &a = pk.a;
        memset(&a, 0, sizeof(a));
        // logical matrix: A is M x K, B is K x N; the K extent is padded to Kp with zeros
        a.rows = (int)(is_a ? p.M : p.K);
        a.cols = (int)(is_a ? p.K : p.N);
        a.contig_cols = is_a ? (orient == 1) : (orient == 0);
        const int64_t rows_x = is_a ? a.rows : Kp, cols_x = is_a ? Kp : a.cols;
        const int64_t rows_p = a.contig_cols ? rows_x : (rows_x + E - 1) / E * E;
        const int64_t cols_p = a.contig_cols ? (cols_x + E - 1) / E * E : cols_x;
        a.rows_p = (int)rows_p;
        a.cols_p = (int)cols_p;
        a.batch = o.bs == 0 ? 1 : (int)p.batch;
        a.src = o.ptr;
        a.s_rs = o.rs; a.s_cs = o.cs; a.s_bs = o.bs;
        a.d_rs = a.contig_cols ? cols_p : 1;
        a.d_cs = a.contig_cols ? 1 : rows_p;
        a.d_bs = o.bs == 0 ? 0 : rows_p * cols_p;
        a.es = es;
        pk.on = true;
        pk.off = ws;
        ws += (rows_p * cols_p * a.batch * es + 255) / 256 * 256;
        o = {placeholder, a.d_rs, a.d_cs, a.d_bs};
        (is_a ? p.a_padded : p.b_padded) = true;
    }
    p.K = Kp;
    return ws;
}

// K slices of a matrix-core plan with `tiles` output tiles: an explicit request, or under the
// AUTO backend enough slices for ~2 workgroups per CU when the tiles alone leave CUs idle (K
// slices of >= 4 stages, at most 64).
int64_t auto_splits(const Prob &p, int64_t tiles, int bk) {
    if (p.split_req > 1) return p.split_req;
    const int cus = dev_info().cus;
    if (p.split_req != 0 || p.backend != MB_BACKEND_AUTO || tiles >= cus || p.K < 2048) return 1;
    int64_t s = (2LL * cus + tiles - 1) / tiles;
    const int64_t maxs = p.K / (4 * bk);
    if (s > maxs) s = maxs;
    if (s > 64) s = 64;
    return s < 1 ? 1 : s;
}

void plan_mfma(const Prob &p, Plan &pl, bool a_kc, bool b_kc, bool thin_ok = false) {
    const int cus = dev_info().cus;
    MfmaTile t;
    bool thin = false;   // the thin-problem tiles below (split for two workgroups per CU)
    bool deepk = false;  // the deep-K schedule (split for one workgroup per CU)
    // a tile in the descriptor is honoured for the matrix-core backends and for AUTO (where
    // the autotuner puts the tile it measured fastest)
    const bool forced = p.tile[0] > 0 && p.tile[1] > 0;
    if (forced) {
        t = snap_tile(p.dt, p.tile, a_kc, b_kc, thin_ok);
    } else if (p.dt == MB_DTYPE_BF16 || p.dt == MB_DTYPE_F16 || p.dt == MB_DTYPE_I8 || p.dt == MB_DTYPE_U8) {
        // Cost model over the LDS-direct 16-bit tiles, in units of one CU's matrix-core time
        // at the ping-pong kernel's rate (~4.8 TFLOP/s per CU, bf16): rounds x tiles resident
        // per CU x BM*BN*K_slice / eff, plus the split-K reduction (partial planes written and
        // read at ~5 TB/s, and a launch).  occ = workgroups per CU (LDS/VGPR limited); eff =
        // relative per-CU throughput, measured on MI355X (bf16 8192^3, 4096^3, 2048^2 x 4096,
        // 1024^2 x 8192, 4096 x 1024 x 4096; 256 x 128 against 128 x 128 on 2048 x 4096 x 2048
        // and 8192 x 1024 x 1024, where 128 x 128 is 4-6 % faster).
        struct Cand {
            MfmaTile t;
            int occ;
            double eff;
        };
        static const Cand cands[] = {
            {{256, 256, 2, 4, 1}, 1, 1.00}, {{256, 128, 2, 4, 1}, 1, 0.90}, {{256, 256, 2, 2}, 1, 0.85},
            {{256, 128, 2, 2}, 1, 0.66},
            {{128, 256, 2, 2}, 1, 0.66}, {{128, 128, 2, 2}, 1, 0.70}, {{128, 64, 2, 2}, 2, 0.65},
            {{64, 128, 2, 2}, 2, 0.60},  {{64, 64, 2, 2}, 3, 0.40},
        };
        const int bk = 128 / dtype_size(p.dt);
        double best = 1e300;
        t = {64, 64, 2, 2};
        for (const auto &c : cands) {
            if (!mfma_tile_compiled(p.dt, c.t)) continue;   // the 256 x 128 ping-pong is 16-bit float only
            const int64_t tiles = ((p.M + c.t.bm - 1) / c.t.bm) * ((p.N + c.t.bn - 1) / c.t.bn) * p.batch;
            const int64_t s = auto_splits(p, tiles, bk);
            // the 256 x 128 ping-pong tile only unsplit: split over K it measured slower than
            // the 128 x 128 tile (2056 x 2048 x 4096: 80.8 us at 4 slices against 51.4)
            if (c.t.sched == 1 && c.t.bn == 128 && s > 1) continue;
            const int64_t wgs = tiles * s, slots = (int64_t)cus * c.occ;
            const int64_t rounds = (wgs + slots - 1) / slots;
            const int64_t per_cu = std::min<int64_t>(c.occ, (wgs + cus - 1) / cus);
            const int64_t kc = (p.K + s - 1) / s;
            double cost = (double)rounds * per_cu * c.t.bm * c.t.bn * (double)kc / c.eff;
            if (s > 1) cost += (double)s * p.M * p.N * p.batch * 3.84 + 7.2e6;
            if (cost < best * 0.999) {
                best = cost;
                t = c.t;
            }
        }
        // Thin problems (fewer 128 x 128 tiles than CUs, deep K, bf16/fp16) where the pick
        // above runs at most one workgroup per CU: 64 x 128 tiles (128 x 64 when M > N), split
        // over K (slices of >= 1024) to two workgroups per CU when the tiles alone do not fill
        // the CUs.  Measured on MI355X, us (cost-model pick -> this): 256x4096x4096 31.5 -> 23.1,
        // 8192x128x4096 31.9 -> 23.7, 128x8192x4096 29.2 -> 25.2, 512x4096x4096 36.2 -> 30.6.
        const int64_t tiles_t = ((p.M + t.bm - 1) / t.bm) * ((p.N + t.bn - 1) / t.bn) * p.batch;
        if ((p.dt == MB_DTYPE_BF16 || p.dt == MB_DTYPE_F16) && p.backend == MB_BACKEND_AUTO && p.split_req == 0 &&
            p.K >= 2048 && ((p.M + 127) / 128) * ((p.N + 127) / 128) * p.batch < cus &&
            tiles_t * auto_splits(p, tiles_t, bk) <= cus) {
            t = p.M > p.N ? MfmaTile{128, 64, 2, 2} : MfmaTile{64, 128, 2, 2};
            thin = true;
        }
        // Deep-K products (bf16 / fp16, at most 64 output tiles of 64 x 64, K >= 8192): the
        // deep-K schedule of the 64 x 64 tile, over K slices of >= 1024 that bring the grid to
        // about one workgroup per CU.  Measured on MI355X, fp16 128 x 128 x 65536 (64 slices):
        // 11.4 us for the kernel plus the reduction of its 64 fp32 planes, against 16.2 us for
        // the rule above (64 x 128 tiles, 64 slices, two LDS buffers).
        const int64_t t64 = ((p.M + 63) / 64) * ((p.N + 63) / 64) * p.batch;
        if ((p.dt == MB_DTYPE_BF16 || p.dt == MB_DTYPE_F16) && p.backend == MB_BACKEND_AUTO && p.split_req == 0 &&
            p.K >= 8192 && p.M > 16 && p.N > 16 && t64 <= 64 && std::min<int64_t>(cus / t64, p.K / 1024) >= 2) {
            t = MfmaTile{64, 64, 2, 2, 2};
            deepk = true;
            thin = false;
        }
    } else {
        static const MfmaTile order[] = {{256, 256, 2, 2}, {256, 128, 2, 2}, {128, 256, 2, 2},
                                         {128, 128, 2, 2}, {128, 64, 2, 2},  {64, 128, 2, 2},
                                         {64, 64, 2, 2}};
        t = {32, 32, 1, 1};
        for (const auto &o : order) {
            const int64_t tiles = ((p.M + o.bm - 1) / o.bm) * ((p.N + o.bn - 1) / o.bn) * p.batch;
            if (tiles >= cus) {
                t = o;
                break;
            }
        }
        if (t.bm == 32) {
            // too few tiles for the big shapes: smallest 4-wave tile unless the problem is tiny
            const int64_t t64 = ((p.M + 63) / 64) * ((p.N + 63) / 64) * p.batch;
            if (t64 >= 16 || p.K >= 1024) t = {64, 64, 2, 2};
        }
    }
    GemmArgs &g = pl.gg;
    fill_gemm_args(p, g);
    const int es = dtype_size(p.dt);
    const int BK = 8 * (16 / es);
    const int64_t tiles = ((p.M + t.bm - 1) / t.bm) * ((p.N + t.bn - 1) / t.bn) * p.batch;
    int64_t splits = auto_splits(p, tiles, BK);
    if (deepk) {
        splits = std::min<int64_t>(cus / tiles, p.K / 1024);
    } else if (thin) {
        splits = 1;
        if (tiles < cus) {
            splits = (2LL * cus + tiles - 1) / tiles;
            const int64_t maxs = p.K / 1024;
            if (splits > maxs) splits = maxs;
            if (splits > 64) splits = 64;
            if (splits < 1) splits = 1;
        }
    }
    if (splits > 1) {
        int64_t chunk = (p.K + splits - 1) / splits;
        chunk = (chunk + BK - 1) / BK * BK;
        splits = (p.K + chunk - 1) / chunk;
        g.k_chunk = (int)chunk;
    }
    g.splits = (int)splits;
    if (splits > 1) pl.ws_bytes = splits * p.batch * p.M * p.N * acc_size(p.dt);
    const int64_t tiles_m = (p.M + t.bm - 1) / t.bm;
    int swz = p.swz;
    if (swz < 0) swz = tiles_m >= 8 ? 3 : ilog2_floor(tiles_m > 0 ? tiles_m : 1);
    if (swz > 6) swz = 6;
    g.swz = swz;
    // vector stores: C row-major, 4-element groups aligned
    g.vec_ok = p.c.cs == 1 && (p.c.rs % 4) == 0 && aligned(p.c.ptr, 4 * es) &&
               (p.batch == 1 || (p.c.bs % 4) == 0);
    // Chained batch entries (k_gemm16): a K slice of at most four stages over many batch
    // entries runs on fewer z-blocks, each workgroup streaming the stages of several entries
    // through its two LDS buffers so that one entry's first loads overlap the previous entry's
    // last stage and epilogue; about four workgroups per CU remain.  Only 16-bit tiles of at
    // most 128 x 128 whose staged output fits one operand stage chain (k_gemm16's CHAIN).
    const bool f16_family = p.dt == MB_DTYPE_BF16 || p.dt == MB_DTYPE_F16;
    if (f16_family && t.sched == 0 && t.bm >= 64 && t.bn >= 64 && t.bm * t.bn <= 128 * 128 && g.k_chunk <= 4 * BK &&
        p.batch > 1 &&
        (int64_t)t.bm * (t.bn * es + 16) <= (int64_t)(t.bm + t.bn) * 128) {
        const int64_t per = std::min<int64_t>(tiles * splits / (4LL * cus), 16);
        if (per >= 2) g.zblocks = (int)((p.batch + per - 1) / per);
    }
    pl.family = MB_FAMILY_MFMA;
    pl.tile = t;
    pl.a_kc = a_kc;
    pl.b_kc = b_kc;
}

void plan_generic(const Prob &p, Plan &pl) {
    GemmArgs &g = pl.gg;
    fill_gemm_args(p, g);
    const int cus = dev_info().cus;
    auto ntiles = [&p](int64_t bt) { return ((p.M + bt - 1) / bt) * ((p.N + bt - 1) / bt) * p.batch; };
    const int64_t tiles = ntiles(64);
    int64_t splits = 1;
    pl.gen_bt = 64;
    if (p.split_req > 1) {
        splits = p.split_req;
    } else if (p.split_req == 0 && tiles < cus && p.K <= 1024 && ntiles(16) >= cus) {
        // few 64 x 64 tiles, short K: 32 x 32 or 16 x 16 tiles fill the CUs with no K slices,
        // so no partial planes and no reduction launch (int32 256^3: 256 tiles of 16 x 16)
        pl.gen_bt = ntiles(32) >= cus ? 32 : 16;
    } else if (p.split_req == 0 && tiles < cus && p.K >= 128) {
        // few output tiles: K slices of >= 16 (one LDS step) so that ~2 workgroups run per CU
        // (int32 256^3: 16 tiles x 16 slices instead of 16 workgroups looping over K)
        splits = (2LL * cus + tiles - 1) / tiles;
        const int64_t maxs = p.K / 16;
        if (splits > maxs) splits = maxs;
        if (splits > 64) splits = 64;
        if (splits < 1) splits = 1;
    }
    if (splits > 1) {
        int64_t chunk = (p.K + splits - 1) / splits;
        chunk = (chunk + 15) / 16 * 16;
        splits = (p.K + chunk - 1) / chunk;
        g.k_chunk = (int)chunk;
        pl.ws_bytes = splits * p.batch * p.M * p.N * acc_size(p.dt);
    }
    g.splits = (int)splits;
    pl.family = MB_FAMILY_GENERIC;
}

// A plan that uses no workspace: one K slice.
void drop_splits(Plan &pl) {
    pl.ws_bytes = 0;
    pl.split_off = 0;
    if (pl.family == MB_FAMILY_GEMV_AXPY) {
        pl.gv.splits = 1;
        pl.gv.k_chunk = pl.gv.K;
    } else {
        pl.gg.splits = 1;
        pl.gg.k_chunk = pl.gg.K;
    }
}

// Complex GEMM on the real matrix cores: C = A @ B as the real product of A's interleaved
// storage (M x 2K) with B expanded into 2 x 2 real blocks (2K x 2N, CplxExpandArgs), i.e. the
// four real products P = Re A Re B, Q = Im A Im B, S = Re A Im B, T = Im A Re B of
// metalblas/complex_dispatch.py:69-81 fused into one GEMM whose output columns interleave
// Re C = P - Q and Im C = S + T (shaders/complex_pack.h:41-42).  Conjugation becomes signs in
// the expansion.  complex64 runs on the fp32 matrix cores, complex32 on fp16 ones (fp32
// accumulation).  Without an epilogue and with row-contiguous C the real GEMM writes C
// directly; otherwise it writes fp32 planes and the split-K reduction, run as complex,
// applies alpha/beta (shaders/complex_pack.h:43-58) and C's strides.
bool plan_complex(const Prob &p, Plan &pl) {
    const bool c64 = p.dt == MB_DTYPE_C64;
    const int res = c64 ? 4 : 2;   // real element bytes
    const int E = 16 / res;
    const char *placeholder = (const char *)(uintptr_t)4096;
    int64_t ws = 0;
    Prob q = p;
    q.dt = c64 ? F32 : F16;
    q.N = 2 * p.N;
    q.K = 2 * p.K;
    q.conj_a = q.conj_b = 0;
    q.epilogue = 0;
    q.beta_nz = 0;
    q.alpha_nz = 1;
    q.bias = {nullptr, 0, 0, 0};
    q.a_padded = q.b_padded = false;
    // A: the interleaved storage read as a real K-contiguous matrix, or a complex copy
    bool view_ok = p.a.cs == 1;
    if (view_ok) {
        q.a = {p.a.ptr, 2 * p.a.rs, 1, 2 * p.a.bs};
        view_ok = operand_ok(q.a, 1, true, q);
    }
    if (!view_ok) {
        PackOp &pk = pl.pack[0];
        PackArgs &a = pk.a;
        memset(&a, 0, sizeof(a));
        const int64_t cols_p = (p.K + E / 2 - 1) / (E / 2) * (E / 2);   // real row length % E == 0
        a.rows = a.rows_p = (int)p.M;
        a.cols = (int)p.K;
        a.cols_p = (int)cols_p;
        a.contig_cols = 1;
        a.batch = p.a.bs == 0 ? 1 : (int)p.batch;
        a.src = p.a.ptr;
        a.s_rs = p.a.rs; a.s_cs = p.a.cs; a.s_bs = p.a.bs;
        a.d_rs = cols_p; a.d_cs = 1;
        a.d_bs = p.a.bs == 0 ? 0 : p.M * cols_p;
        a.es = dtype_size(p.dt);
        pk.on = true;
        pk.off = ws;
        ws += (p.M * cols_p * a.batch * a.es + 255) / 256 * 256;
        q.a = {placeholder, 2 * cols_p, 1, 2 * a.d_bs};
        q.a_padded = true;
    }
    // B: expanded into the workspace, K-contiguous, K zero-padded to a 16-byte multiple
    CplxExpandArgs &cx = pl.cx;
    memset(&cx, 0, sizeof(cx));
    const int64_t ldb = (2 * p.K + E - 1) / E * E;
    cx.b = p.b.ptr;
    cx.b_rs = p.b.rs; cx.b_cs = p.b.cs; cx.b_bs = p.b.bs;
    cx.ld = ldb;
    cx.K = (int)p.K;
    cx.N = (int)p.N;
    cx.batch = p.b.bs == 0 ? 1 : (int)p.batch;
    cx.d_bs = p.b.bs == 0 ? 0 : 2 * p.N * ldb;
    cx.neg_a = p.conj_a;
    cx.neg_b = p.conj_b;
    cx.half = !c64;
    pl.cx_off = ws;
    ws += (2 * p.N * ldb * cx.batch * res + 255) / 256 * 256;
    q.b = {placeholder, 1, ldb, cx.d_bs};
    q.b_padded = true;
    // C: written directly when the real view is plain, else fp32 planes + complex reduction
    const bool direct = !p.epilogue && p.c.cs == 1;
    q.c = direct ? Operand{p.c.ptr, 2 * p.c.rs, 1, 2 * p.c.bs} : Operand{placeholder, q.N, 1, p.M * q.N};
    bool a_kc = false, b_kc = false;
    if (!mfma_layout_ok(q, a_kc, b_kc)) {
        pl.pack[0] = PackOp();
        return false;
    }
    plan_mfma(q, pl, a_kc, b_kc);
    GemmArgs &g = pl.gg;
    pl.split_off = ws;
    if (direct) {
        pl.ws_bytes += ws;   // split-K planes, if any, after the copies
    } else {
        g.planes = 1;
        pl.ws_bytes = ws + (int64_t)g.splits * p.batch * p.M * q.N * 4;
        GemmArgs &r = pl.cr;
        memset(&r, 0, sizeof(r));
        r.c = (void *)p.c.ptr;
        r.bias = p.bias.ptr;
        r.M = (int)p.M; r.N = (int)p.N; r.batch = (int)p.batch;
        r.c_rs = p.c.rs; r.c_cs = p.c.cs; r.c_bs = p.c.bs;
        r.bias_rs = p.bias.rs; r.bias_cs = p.bias.cs; r.bias_bs = p.bias.bs;
        r.epilogue = p.epilogue; r.beta_nz = p.beta_nz; r.alpha_nz = p.alpha_nz;
        r.s = p.s;
        pl.cplx_reduce = true;
    }
    pl.cplx = true;
    pl.cdt = p.dt;
    pl.p = q;
    return true;
}

// Products with a few vectors (up to 32; one only against a mid-size N-contiguous matrix) and a
// large matrix run on the matrix cores, which read the matrix once at HBM speed whatever the
// vector count (the VALU GEMV kernels spend nv FMAs per matrix element, which outgrows the HBM
// stream from about 4 vectors up).  Thin tiles:
//   4 x 8    (k_dotx):     matrix = A, K-contiguous; up to 8 vectors = columns of B, whole K;
//   4 x 16   (k_thin_dot4) and 64 x 16 (k_thin_dot): matrix = A, K-contiguous, K slices;
//   32 x 256, 32 x 128 (k_thin16): matrix = B, N-contiguous; vectors = rows of A.
// The other two layouts are the transposed problem of these.  The vectors must be
// K-contiguous and are copied (nv x K elements) when they are not; a matrix the loaders cannot
// stream in place is left to the GEMV path.  K is split when the tiles alone leave CUs idle.
// bf16 / fp16 only.
// Measured on MI355X (bf16, 16384^2 matrix): the 32 x 256 tile streams at ~92 us for every
// vector count from 2 up (VALU: 95 us at 2 vectors, 118 at 8, 189 at 16); k_thin_dot4 at
// ~111 us (VALU: 95-97 us at 2 and 4 vectors, 347 at 3, 195 at 8, 624 at 16).
constexpr int kThinMfmaMinNvDot = 5;

bool plan_thin_mfma(const Prob &p, Plan &pl) {
    if (p.dt != MB_DTYPE_BF16 && p.dt != MB_DTYPE_F16) return false;
    MfmaTile req = {0, 0, 0, 0, 0};
    if (p.tile[0] > 0 && p.tile[1] > 0) {   // an explicit tile: only a thin one keeps this plan
        req = {p.tile[0], p.tile[1], 0, 0, 0};
        if (!thin_tile(req)) return false;
    }
    const bool vec_b = p.N <= p.M;   // vectors are the columns of B
    const int64_t nv = vec_b ? p.N : p.M, wide = vec_b ? p.M : p.N;
    const int mo = vec_b ? a_orient(p) : b_orient(p);   // the matrix: 1 = K-contiguous
    if (mo < 0) return false;
    // the dot tiles take up to 16 vectors, the 32 x 256 tile up to 32
    if (nv > (mo == 1 ? 16 : 32)) return false;
    if (req.bm == 0) {   // the automatic choice (an explicit thin tile skips these)
        if (mo == 1) {
            if (nv > 16 || wide < 2048 || p.K < 2048) return false;
            // K-contiguous matrix: the VALU kernels stream 2 and 4 vectors faster (95-97 us vs
            // ~111 us); 3 vectors have no fast VALU form (347 us)
            if (nv < kThinMfmaMinNvDot && nv != 3) return false;
        } else {
            // one vector (x @ W): the tile's stream needs no K-slice planes when the columns
            // fill the CUs, and wins below ~0.4 GB of matrix; above it the VALU stream's longer
            // runs win.  Measured on MI355X (bf16, us, VALU -> thin tile): 4096^2 19.0 -> 11.9,
            // 32000 x 4096 46.4 -> 43.8, 65536 x 2048 45.5 -> 42.4; kept: 16384^2 82.0 (85.4),
            // 32000 x 8192 82.4 (84.8).
            const int64_t mat1 = wide * p.K * p.batch * dtype_size(p.dt);
            if (nv == 1 && (mat1 < (32LL << 20) || mat1 >= (384LL << 20) || (wide + 255) / 256 * p.batch < 8))
                return false;
            // N-contiguous matrix on the 32 x 256 tile.  Up to 16 vectors: a large matrix
            // (>= 32 MiB over >= 8 tiles), also with a short K or a batch, where the VALU
            // kernel's K slices write fp32 planes of nv x N per slice.  17-32 vectors (where
            // the alternative is the 64 x 128 tile with half its rows idle): a matrix of
            // >= 256 MiB, or enough tiles for every CU without K slices.  Measured on MI355X
            // (bf16, us, VALU or 64 x 128 -> 32 x 256): 16 x 65536 x 1024 71.6 -> 22.5,
            // bmm 64 x 16 x 4096 x 512 109 -> 60, 512 x 16 x 1024 x 512 316 -> 101,
            // 32 x 16384^2 104 -> 89, bmm 256 x 32 x 2048 x 512 116 -> 107; kept:
            // 32 x 8192^2 29.7 (34.0), 32 x 16384 x 4096 27.5 (31.1).
            const int64_t tiles = (wide + 255) / 256 * p.batch;
            const int64_t mat_bytes = wide * p.K * p.batch * dtype_size(p.dt);
            const bool take = nv <= 16 ? (wide >= 2048 && p.K >= 2048) || (mat_bytes >= (32LL << 20) && tiles >= 8)
                                       : mat_bytes >= (256LL << 20) || tiles >= dev_info().cus;
            if (!take) return false;
        }
    }
    Prob q = p;
    if ((mo == 1) != vec_b) transpose(q);   // K-contiguous matrix as A, N-contiguous as B
    const bool dot = mo == 1;
    const int64_t cus = dev_info().cus;
    // k_dotx: up to 8 vectors and K <= 16384 over the whole K in one workgroup (no K slices,
    // no reduction), when its 16-quad groups alone give every CU a workgroup (or on request);
    // the vectors stream in place K-contiguous or as the natural 8-wide rows, else they are
    // copied K-contiguous.  Measured on MI355X (bf16, 16384^2 x 8, per call): 85 us with the
    // natural vectors against 99.9 us for k_thin_dot4 (vector copy, 4 K slices, reduction).
    const int64_t groups = ((q.M + 3) / 4 + m16::kDotxQG - 1) / m16::kDotxQG;
    const bool want_dotx = req.bm == 4 && req.bn == 8, want_other = req.bm > 0 && !want_dotx;
    bool dotx = dot && nv <= 8 && q.K % 8 == 0 && q.K <= (int64_t)m16::kDotxMaxWaves * m16::kDotxKW &&
                q.batch <= 65535 && !want_other && (want_dotx || groups * q.batch >= cus);
    const bool natural = dotx && b_orient(q) == 0 && q.N == 8 && operand_ok(q.b, 0, false, q);
    Plan trial;
    // vectors K-contiguous (copied when they are not), except the natural rows of k_dotx
    const int64_t pack_bytes = plan_packs(q, trial, natural ? 0 : (dot ? 2 : 1));
    if (trial.pack[dot ? 0 : 1].on) return false;                    // never copy the matrix
    bool a_kc = false, b_kc = false;
    if (!mfma_layout_ok(q, a_kc, b_kc) || !(dotx ? a_kc : dot ? a_kc && b_kc : a_kc && !b_kc)) return false;
    // the K-contiguous matrix otherwise: k_thin_dot4 (4-row streams) when its 31-bit offsets
    // cover the matrix, else k_thin_dot
    bool dot4 = false;
    if (dot) {
        GemmArgs probe;
        fill_gemm_args(q, probe);
        if (dotx) dotx = m16::dotx_offsets_fit(probe, b_kc);
        if (!dotx) dot4 = m16::thin_dot4_offsets_fit(probe);
    }
    if (natural && !dotx) return false;   // (31-bit offsets only: a matrix of > 1 GiB)
    // the N-contiguous matrix: 32 x 128 (an 80 KiB ring, two workgroups per CU, so one's
    // prologue overlaps the other's stream) when the 32 x 256 tile would stream at most 512 of K
    // per workgroup or split K; else 32 x 256.  Measured on MI355X (bf16, us, 32 x 256 ->
    // 32 x 128): bmm 64 x 8 x 4096 x 512 58.3 -> 47.9, bmm 32 x 16 x 8192 x 256 38.7 -> 29.9,
    // 16 x 16384 x 2048 17.2 -> 15.3, 8 x 16384^2 85.7 -> 85.2; kept: bmm 128 x 16 x 2048 x 1024
    // 88.6 (95.2), 16 x 65536 x 1024 22.5 (23.0).
    int rows_bn = 256;
    if (!dot && !dotx) {
        if (req.bm == 32) {
            rows_bn = req.bn == 128 ? 128 : 256;
        } else {
            const int64_t tiles256 = (q.N + 255) / 256 * q.batch;
            const int64_t max_splits = q.K / (4 * (128 / dtype_size(q.dt)));
            const bool split = q.split_req > 1 || (tiles256 < cus && max_splits > 1);
            if (split || q.K <= 512) rows_bn = 128;
        }
    }
    const MfmaTile t = dotx  ? MfmaTile{4, 8, m16::kDotxMaxWaves, 1, 0}
                       : dot ? (dot4 ? MfmaTile{4, 16, 1, 1, 0} : MfmaTile{64, 16, 4, 1, 0})
                             : MfmaTile{32, rows_bn, 1, 4, 0};
    q.tile[0] = t.bm; q.tile[1] = t.bn; q.tile[2] = 0; q.tile[3] = t.wm; q.tile[4] = t.wn; q.tile[5] = t.sched + 1;
    const int64_t req_split = q.split_req;
    q.split_req = 1;
    pl.pack[0] = trial.pack[0];
    pl.pack[1] = trial.pack[1];
    pl.p = q;
    plan_mfma(q, pl, a_kc, b_kc, true);
    if (pl.tile.bm != t.bm || pl.tile.bn != t.bn) return false;
    if (dot && !dotx && !m16::thin_dot_offsets_fit(pl.gg)) return false;
    // K slices: whole macro steps (512) for k_thin_dot, whole stages for k_thin16, at least
    // two / four of them per slice
    GemmArgs &g = pl.gg;
    int64_t splits;
    if (dotx) {
        splits = 1;
        g.k_chunk = (int)q.K;
        g.persist = (int)groups;
    } else if (dot4) {
        // fixed K slices of m16::kThinDot4Chunk; a persistent grid that walks the row quads, so
        // each workgroup loads its vector slice once: two workgroups per CU, one for matrices
        // of 256 MiB and more.  Measured on MI355X (bf16, 8 vectors, us, two -> one per CU):
        // 16384^2 113.3 -> 101.4, 32768 x 8192 105.7 -> 103.9, 16384 x 16384 x 12 vectors
        // 115.6 -> 110.1; 16384 x 4096 27.9 -> 29.8, 8192^2 (6 vectors) 30.8 -> 32.3.
        splits = (q.K + m16::kThinDot4Chunk - 1) / m16::kThinDot4Chunk;
        g.k_chunk = m16::kThinDot4Chunk;
        const int64_t quads = (q.M + 3) / 4;
        const int64_t per_cu = (int64_t)q.M * q.K * dtype_size(q.dt) >= ((int64_t)256 << 20) ? 1 : 2;
        int64_t wgs = (per_cu * cus + splits * q.batch - 1) / (splits * q.batch);
        g.persist = (int)(wgs < quads ? wgs : quads);
    } else {
        const int64_t unit = dot ? 512 : 128 / dtype_size(q.dt);
        const int64_t tiles = (dot ? (q.M + 63) / 64 : (q.N + t.bn - 1) / t.bn) * q.batch;
        splits = req_split > 0 ? req_split : (cus + tiles - 1) / tiles;
        const int64_t maxs = q.K / ((dot ? 2 : 4) * unit);
        if (req_split <= 0 && splits > maxs) splits = maxs;
        if (splits > 64) splits = 64;
        if (splits < 1) splits = 1;
        int64_t chunk = (q.K + splits - 1) / splits;
        chunk = (chunk + unit - 1) / unit * unit;
        splits = (q.K + chunk - 1) / chunk;
        g.k_chunk = (int)(splits > 1 ? chunk : (dot ? (q.K + 511) / 512 * 512 : q.K));
    }
    g.splits = (int)splits;
    pl.ws_bytes = splits > 1 ? splits * q.batch * q.M * q.N * acc_size(q.dt) : 0;
    pl.split_off = pack_bytes;
    pl.ws_bytes += pack_bytes;
    return true;
}

// allow_ws = false plans without any workspace use: no operand copies and no split-K.
int make_plan(const mb_gemm_desc *d, Plan &pl, bool allow_ws = true) {
    Prob p;
    int st = normalise(d, p);
    if (st != MB_OK) return st;
    pl.family = MB_FAMILY_NONE;
    pl.ws_bytes = 0;
    if (p.batch == 0 || p.M == 0 || p.N == 0) {
        pl.p = p;
        return MB_OK;
    }
    if (p.K == 0) {
        pl.p = p;
        fill_gemm_args(p, pl.gg);
        pl.family = MB_FAMILY_FILL;
        return MB_OK;
    }
    // column-major outputs are produced as the transposed row-major problem
    if (p.c.cs != 1 && p.c.rs == 1) transpose(p);
    pl.p = p;

    if (p.backend == MB_BACKEND_GENERIC) {
        plan_generic(p, pl);
        if (!allow_ws) drop_splits(pl);
        return MB_OK;
    }
    const bool thin = p.M <= 16 || p.N <= 16;
    // an explicit tile-family request (the autotuner's candidate, or matmul(tile=...)) on a
    // product that is not a single vector runs on the matrix cores instead of the GEMV kernels
    const bool tile_req = p.tile[0] > 0 && p.tile[1] > 0 && !thin_tile(MfmaTile{p.tile[0], p.tile[1], 0, 0, 0}) &&
                          p.M > 1 && p.N > 1;
    if (p.backend == MB_BACKEND_AUTO && (p.M <= 32 || p.N <= 32) && allow_ws) {
        Plan tp = pl;
        if (plan_thin_mfma(p, tp)) {
            pl = tp;
            return MB_OK;
        }
    }
    if (p.backend == MB_BACKEND_GEMV || (p.backend == MB_BACKEND_AUTO && thin && !tile_req)) {
        if (plan_gemv(p, pl)) {
            if (!allow_ws) drop_splits(pl);
            return MB_OK;
        }
        if (p.backend == MB_BACKEND_GEMV) {
            // a gemv request whose matrix has no unit stride: generic kernel, same results
            plan_generic(p, pl);
            if (!allow_ws) drop_splits(pl);
            return MB_OK;
        }
    }
    bool a_kc = false, b_kc = false;
    const bool tiny = p.backend == MB_BACKEND_AUTO && p.M < 32 && p.N < 32;
    if ((p.dt == MB_DTYPE_C64 || p.dt == MB_DTYPE_C32) && allow_ws && !tiny &&
        (p.backend == MB_BACKEND_AUTO || p.backend == MB_BACKEND_MATRIX || p.backend == MB_BACKEND_TILED) &&
        (double)p.M * p.N * p.K * p.batch >= (double)(1 << 22)) {
        if (plan_complex(p, pl)) return MB_OK;
    }
    if (mfma_layout_ok(p, a_kc, b_kc) && !tiny) {
        plan_mfma(p, pl, a_kc, b_kc);
        if (!allow_ws) drop_splits(pl);
        return MB_OK;
    }
    // operands the loaders cannot stream: copy them once into the workspace when the product
    // is large enough for the matrix cores to repay the copy (2 x the operand bytes)
    if (allow_ws && mfma_supported_dtype(p.dt) && !tiny &&
        (p.backend == MB_BACKEND_AUTO || p.backend == MB_BACKEND_MATRIX || p.backend == MB_BACKEND_TILED) &&
        (double)p.M * p.N * p.K * p.batch >= (double)(1 << 24)) {
        Prob q = p;
        Plan trial;
        const int64_t pack_bytes = plan_packs(q, trial);
        if (mfma_layout_ok(q, a_kc, b_kc)) {
            pl.pack[0] = trial.pack[0];
            pl.pack[1] = trial.pack[1];
            pl.p = q;
            plan_mfma(q, pl, a_kc, b_kc);
            pl.split_off = pack_bytes;
            pl.ws_bytes += pack_bytes;
            return MB_OK;
        }
    }
    plan_generic(p, pl);
    if (!allow_ws) drop_splits(pl);
    return MB_OK;
}

int run_plan(Plan &pl, const mb_gemm_desc *d, hipStream_t st, LaunchShape *shape) {
    hipError_t e = hipSuccess;
    if (pl.ws_bytes > 0 && (!d->workspace || d->workspace_bytes < pl.ws_bytes)) return MB_ERR_WORKSPACE;
    char *wsb = (char *)d->workspace;
    for (int which = 0; which < 2; ++which)
        if (pl.pack[which].on) pl.pack[which].a.dst = wsb + pl.pack[which].off;
    if (pl.pack[0].on && pl.pack[1].on)
        e = launch_pack2(pl.pack[0].a, pl.pack[1].a, st);
    else if (pl.pack[0].on || pl.pack[1].on)
        e = launch_pack(pl.pack[pl.pack[0].on ? 0 : 1].a, st);
    if (e != hipSuccess) return MB_ERR_LAUNCH;
    if (pl.pack[0].on) pl.gg.a = pl.pack[0].a.dst;
    if (pl.pack[1].on) pl.gg.b = pl.pack[1].a.dst;
    switch (pl.family) {
        case MB_FAMILY_NONE:
            return MB_OK;
        case MB_FAMILY_FILL:
            e = launch_fill(pl.p.dt, pl.gg, st);
            break;
        case MB_FAMILY_GENERIC:
        case MB_FAMILY_MFMA: {
            GemmArgs &g = pl.gg;
            if (pl.cplx) {
                pl.cx.dst = wsb + pl.cx_off;
                e = launch_cplx_expand(pl.cx, st);
                if (e != hipSuccess) break;
                g.b = pl.cx.dst;
            }
            g.ws = wsb ? wsb + pl.split_off : nullptr;
            e = pl.family == MB_FAMILY_MFMA ? launch_mfma(pl.p.dt, pl.tile, pl.a_kc, pl.b_kc, g, st, shape)
                                            : launch_generic(pl.p.dt, pl.gen_bt, g, st, shape);
            if (e != hipSuccess) break;
            if (pl.cplx_reduce) {
                pl.cr.ws = g.ws;
                pl.cr.splits = g.splits;
                e = launch_splitk_reduce(pl.cdt, pl.cr, st);
            } else if (g.splits > 1) {
                e = launch_splitk_reduce(pl.p.dt, g, st);
            }
            break;
        }
        case MB_FAMILY_GEMV_DOT:
            e = pl.gemv_fast ? launch_gemv_dot_fast(pl.p.dt, pl.gv, st, shape)
                             : launch_gemv_dot(pl.p.dt, pl.gv, st, shape);
            break;
        case MB_FAMILY_GEMV_AXPY: {
            GemvArgs &g = pl.gv;
            g.ws = d->workspace;
            e = pl.gemv_fast ? launch_gemv_axpy_fast(pl.p.dt, g, st, shape) : launch_gemv_axpy(pl.p.dt, g, st, shape);
            if (e == hipSuccess && g.splits > 1) {
                // sum the K slices: partial planes are [split][batch][nv][rows]
                GemmArgs r;
                memset(&r, 0, sizeof(r));
                r.ws = g.ws;
                r.c = g.y;
                r.bias = g.bias;
                r.M = g.nv; r.N = g.rows; r.batch = g.batch;
                r.c_rs = g.y_vs; r.c_cs = g.y_is; r.c_bs = g.y_bs;
                r.bias_rs = g.bias_vs; r.bias_cs = g.bias_is; r.bias_bs = g.bias_bs;
                r.epilogue = g.epilogue; r.beta_nz = g.beta_nz; r.alpha_nz = g.alpha_nz;
                r.s = g.s;
                r.splits = g.splits;
                e = launch_splitk_reduce(pl.p.dt, r, st);
            }
            break;
        }
        default:
            return MB_ERR_INVALID_ARG;
    }
    return e == hipSuccess ? MB_OK : MB_ERR_LAUNCH;
}

// The plan one launch sequence runs: the workspace plan, or, when the caller's scratch is
// missing or too small, the plan that needs none (same results).
int plan_one(const mb_gemm_desc *desc, Plan &pl) {
    int st = make_plan(desc, pl);
    if (st != MB_OK) return st;
    if (pl.ws_bytes > 0 && (!desc->workspace || desc->workspace_bytes < pl.ws_bytes)) {
        if (desc->flags & kFlagStaticScratch) return MB_ERR_SCRATCH_LIMIT;
        pl = Plan();
        st = make_plan(desc, pl, false);
    }
    return st;
}

// ---- edge peeling ---------------------------------------------------------------------------
// A bf16/fp16 product whose M (or N) ends 1..16 past a multiple of 256 has a last row (column)
// of tiles that are almost empty yet cost a whole round of matrix-core time: 4097 x 4096 x 4096
// runs 561 256 x 128 tiles in three rounds on 256 CUs.  It runs as the core [0, M') x [0, N')
// on whole 256 x 256 tiles plus the 1..16-row (column) strips on the GEMV or thin kernels: up
// to three launches on the caller's stream, one after another, sharing the workspace.  Taken
// only when the core runs 256 x 256 tiles over K >= 2048, every strip runs on a streaming
// kernel (fast GEMV or a thin matrix-core tile) and the core copies no operand that the whole
// product would not copy too.  Measured on MI355X (bf16, us, best whole-product tile ->
// peeled; hipBLASLt): 4097 x 4096 x 4096 162.1 -> 117.2 (124.2), 2056 x 8192 x 4096 160.2 ->
// 119.8 (125.8), 4096 x 4100 x 4096 185.7 -> 149.1 (134.2), 4097 x 4096 x 2048 85.9 -> 72.3
// (67.5), 8200 x 8192 x 8192 900.3 -> 797.4 (864.9).  Smaller cores lose: 2049 x 2048 x 2048
// on 128 x 128 tiles 30.1 -> 36.3 (the strip's launch costs more than the tiles save), and
// 8193 x 8192 x 1024 153.4 -> 157.6.
struct Peel {
    int n = 0;
    mb_gemm_desc part[3];
};

bool streaming_plan(const Plan &pl) {
    if (pl.family == MB_FAMILY_GEMV_DOT || pl.family == MB_FAMILY_GEMV_AXPY) return pl.gemv_fast;
    return pl.family == MB_FAMILY_MFMA && thin_tile(pl.tile);
}

bool plan_peel(const mb_gemm_desc *d, Peel &pe) {
    if (d->backend != MB_BACKEND_AUTO || d->batch != 1 || d->split_k != 0 || d->tile[0] > 0 || d->tile[1] > 0)
        return false;
    if (d->dtype != MB_DTYPE_BF16 && d->dtype != MB_DTYPE_F16) return false;
    if (d->M < 2048 || d->N < 2048 || d->K < 2048) return false;
    const int64_t rm = d->M % 256, rn = d->N % 256;
    const bool pm = rm >= 1 && rm <= 16, pn = rn >= 1 && rn <= 16;
    if (!pm && !pn) return false;
    const int64_t mm = d->M - (pm ? rm : 0), nn = d->N - (pn ? rn : 0);
    const int64_t es = dtype_size(d->dtype);
    auto at = [es](void *ptr, int64_t elems) { return ptr ? (void *)((char *)ptr + elems * es) : ptr; };
    pe.n = 0;
    mb_gemm_desc core = *d;
    core.M = mm;
    core.N = nn;
    pe.part[pe.n++] = core;
    if (pm) {   // rows [mm, M) x all N
        mb_gemm_desc s = *d;
        s.M = rm;
        s.a.ptr = at(d->a.ptr, mm * d->a.row_stride);
        s.c.ptr = at(d->c.ptr, mm * d->c.row_stride);
        s.bias.ptr = at(d->bias.ptr, mm * d->bias.row_stride);
        pe.part[pe.n++] = s;
    }
    if (pn) {   // rows [0, mm) x columns [nn, N)
        mb_gemm_desc s = *d;
        s.M = mm;
        s.N = rn;
        s.b.ptr = at(d->b.ptr, nn * d->b.col_stride);
        s.c.ptr = at(d->c.ptr, nn * d->c.col_stride);
        s.bias.ptr = at(d->bias.ptr, nn * d->bias.col_stride);
        pe.part[pe.n++] = s;
    }
    Plan whole, pc;
    if (make_plan(d, whole) != MB_OK || make_plan(&pe.part[0], pc) != MB_OK) return false;
    if (pc.family != MB_FAMILY_MFMA || pc.tile.bm != 256 || pc.tile.bn != 256) return false;
    if ((pc.pack[0].on && !whole.pack[0].on) || (pc.pack[1].on && !whole.pack[1].on)) return false;
    for (int i = 1; i < pe.n; ++i) {
        Plan ps;
        if (make_plan(&pe.part[i], ps) != MB_OK || !streaming_plan(ps)) return false;
    }
    return true;
}

// ---- per-signature plan cache ---------------------------------------------------------------
// Planning a call (normalisation, the tile cost model, the peeling trial) takes 4-20 us of host
// time, as long as a small product's kernel.  A plan depends on the operand pointers only
// through null-ness and alignment (every check is modulo 64 bytes or less), so mb_gemm plans
// each call signature once, on sentinel pointers that keep each real pointer's low 8 bits, and
// later calls relocate the cached plan's pointer fields from the sentinels to their own
// operands.  The signature is the whole descriptor with the pointers so replaced, the workspace
// reduced to present / absent, and the current device.  METALBLAS_LAUNCH_CACHE=0 turns the cache
// off; METALBLAS_LAUNCH_CACHE=verify also replans every hit from the real descriptor and aborts
// when a relocated pointer or a launch choice differs.

constexpr uint64_t kSentBase = uint64_t(1) << 56;   // above every canonical host / HSA address
constexpr uint64_t kSentSpan = uint64_t(1) << 52;   // one span per operand: a, b, c, bias
// spans 4..6: the workspace copies of a packed peel (placed at run time)
constexpr uint64_t kSentCopy = kSentBase + 4 * kSentSpan;

struct CallPlan {
    int n = 0;       // launch sequences: 1, or the 2-3 parts of a peeled product
    Plan part[3];
    int ncopy = 0;   // packed peel: operand copies made before the parts
    PackOp copy[3];  // (their .off is the workspace offset; the parts' workspace follows)
    int64_t copy_bytes = 0;
};

// ---- packed peel ------------------------------------------------------------------------------
// A product whose operands are both copied anyway (rows no loader can stream in place: an odd
// K, a storage offset) and whose M or N ends 1..16 past a multiple of 256 (4097^3: 17 x 33
// tiles of 256 x 128 in three rounds) is peeled after the copies: A and B are copied once,
// row-major with K zero-padded to a whole stage (aligned rows), B's last 1..16 columns also
// K-contiguous, and the core runs whole 256 x 256 tiles on the copies while the strips stream
// them on the fast GEMV or thin kernels, all on the caller's stream: rows [M', M) x columns
// [0, N') and all rows x columns [N', N) (the corner with the columns).  The copies take the front
// of the workspace; the parts are planned on sentinel pointers for them (spans 4..6), which
// gemm_impl places.  Row-major A and B (unit column stride), batch 1, bf16 / fp16, the AUTO
// backend, no tile or split request.
bool plan_packed_peel(const mb_gemm_desc *d, CallPlan &cp, bool sizing) {
    if (d->backend != MB_BACKEND_AUTO || d->batch != 1 || d->split_k != 0 || d->tile[0] > 0 || d->tile[1] > 0)
        return false;
    if (d->dtype != MB_DTYPE_BF16 && d->dtype != MB_DTYPE_F16) return false;
    if (d->M < 2048 || d->N < 2048 || d->K < 2048 || d->a.col_stride != 1 || d->b.col_stride != 1) return false;
    if (d->conj_a || d->conj_b) return false;
    if (!sizing && !d->workspace) return false;
    const int64_t rm = d->M % 256, rn = d->N % 256;
    const bool pm = rm >= 1 && rm <= 16, pn = rn >= 1 && rn <= 16;
    if (!pm && !pn) return false;
    Plan whole;
    if (make_plan(d, whole) != MB_OK || whole.family != MB_FAMILY_MFMA || !whole.pack[0].on || !whole.pack[1].on)
        return false;
    const int es = dtype_size(d->dtype);
    const int64_t mm = d->M - (pm ? rm : 0), nn = d->N - (pn ? rn : 0);
    const int64_t Kp = (d->K + 128 / es - 1) / (128 / es) * (128 / es);   // whole 128-byte stages
    const int64_t Np = (d->N + 16 / es - 1) / (16 / es) * (16 / es);      // 16-byte rows
    auto copy_op = [&](const void *src, int64_t s_rs, int64_t s_cs, int64_t rows, int64_t cols, int64_t rows_p,
                       int64_t cols_p, bool contig_cols, int64_t &off) {
        PackOp pk;
        PackArgs &a = pk.a;
        memset(&a, 0, sizeof(a));
        a.src = src;
        a.s_rs = s_rs; a.s_cs = s_cs;
        a.rows = (int)rows; a.cols = (int)cols; a.rows_p = (int)rows_p; a.cols_p = (int)cols_p;
        a.contig_cols = contig_cols;
        a.d_rs = contig_cols ? cols_p : 1;
        a.d_cs = contig_cols ? 1 : rows_p;
        a.batch = 1;
        a.es = es;
        pk.on = true;
        pk.off = off;
        off += (rows_p * cols_p * es + 255) / 256 * 256;
        return pk;
    };
    int64_t off = 0;
    cp.ncopy = 0;
    // A: M x Kp row-major; B: Kp x Np row-major; B's columns [nn, N): K-contiguous, rn x Kp
    cp.copy[cp.ncopy++] = copy_op(d->a.ptr, d->a.row_stride, 1, d->M, d->K, d->M, Kp, true, off);
    cp.copy[cp.ncopy++] = copy_op(d->b.ptr, d->b.row_stride, 1, d->K, d->N, Kp, Np, true, off);
    if (pn)
        cp.copy[cp.ncopy++] = copy_op((const char *)d->b.ptr + nn * es, d->b.row_stride, 1, d->K, rn, Kp, rn, false, off);
    cp.copy_bytes = off;
    const int64_t avail = sizing ? (int64_t(1) << 50) : d->workspace_bytes - off;
    if (avail < 0) return false;
    auto sent = [es](int k, int64_t elems) { return (void *)(uintptr_t)(kSentCopy + (uint64_t)k * kSentSpan + elems * es); };
    auto at = [es](void *ptr, int64_t elems) { return ptr ? (void *)((char *)ptr + elems * es) : ptr; };
    mb_gemm_desc base = *d;
    base.K = Kp;
    base.a = {sent(0, 0), Kp, 1, 0};
    base.b = {sent(1, 0), Np, 1, 0};
    base.workspace = sizing ? (void *)(uintptr_t)1 : d->workspace;
    base.workspace_bytes = avail;
    mb_gemm_desc part[3];
    int n = 0;
    part[n] = base;
    part[n].M = mm;
    part[n].N = nn;
    ++n;
    if (pm) {   // rows [mm, M) x columns [0, nn) (8-aligned rows for the x @ W stream)
        part[n] = base;
        part[n].M = rm;
        part[n].N = nn;
        part[n].a.ptr = sent(0, mm * Kp);
        part[n].c.ptr = at(d->c.ptr, mm * d->c.row_stride);
        part[n].bias.ptr = at(d->bias.ptr, mm * d->bias.row_stride);
        ++n;
    }
    if (pn) {   // all rows x columns [nn, N), against the K-contiguous column copy
        part[n] = base;
        part[n].N = rn;
        part[n].b = {sent(2, 0), 1, Kp, 0};
        part[n].c.ptr = at(d->c.ptr, nn * d->c.col_stride);
        part[n].bias.ptr = at(d->bias.ptr, nn * d->bias.col_stride);
        ++n;
    }
    for (int i = 0; i < n; ++i)
        if (plan_one(&part[i], cp.part[i]) != MB_OK) return false;
    const Plan &pc = cp.part[0];
    if (pc.family != MB_FAMILY_MFMA || pc.tile.bm != 256 || pc.tile.bn != 256 || pc.pack[0].on || pc.pack[1].on)
        return false;
    for (int i = 1; i < n; ++i)
        if (!streaming_plan(cp.part[i]) || cp.part[i].pack[0].on || cp.part[i].pack[1].on) return false;
    cp.n = n;
    return true;
}

int plan_call(const mb_gemm_desc *d, CallPlan &cp, bool sizing = false) {
    Peel pe;
    if (plan_peel(d, pe)) {
        cp.n = pe.n;
        for (int i = 0; i < pe.n; ++i) {
            const int st = plan_one(&pe.part[i], cp.part[i]);
            if (st != MB_OK) return st;
        }
        return MB_OK;
    }
    {
        CallPlan pp;
        if (plan_packed_peel(d, pp, sizing)) {
            cp = pp;
            return MB_OK;
        }
    }
    cp = CallPlan();
    cp.n = 1;
    return plan_one(d, cp.part[0]);
}

// the workspace a call plan needs: its copies, then the largest part's own workspace (the
// parts run one after another)
int64_t call_ws_bytes(const CallPlan &cp) {
    int64_t ws = 0;
    for (int i = 0; i < cp.n; ++i) ws = std::max<int64_t>(ws, cp.part[i].ws_bytes);
    return cp.copy_bytes + ws;
}

// Calls f on every device pointer a plan holds (all are copies of, or offsets into, the
// descriptor's a / b / c / bias operands, or set from the workspace at run time).
template <class F>
void each_ptr(Plan &pl, F f) {
    f(pl.p.a.ptr); f(pl.p.b.ptr); f(pl.p.c.ptr); f(pl.p.bias.ptr);
    for (PackOp &pk : pl.pack) { f(pk.a.src); f(pk.a.dst); }
    f(pl.cx.b); f(pl.cx.dst);
    for (GemmArgs *g : {&pl.cr, &pl.gg}) { f(g->a); f(g->b); f(g->c); f(g->bias); f(g->ws); }
    f(pl.gv.mat); f(pl.gv.x); f(pl.gv.y); f(pl.gv.bias); f(pl.gv.ws);
}

struct Reloc {
    uint64_t sent[4], real[4];
};

template <class T>
void relocate(T *&ptr, const Reloc &r) {
    const uint64_t v = (uint64_t)(uintptr_t)ptr;
    const uint64_t lo = kSentBase - kSentSpan / 2;
    if (v < lo || v >= lo + 4 * kSentSpan) return;   // not derived from an operand
    const int k = (int)((v - lo) / kSentSpan);
    ptr = (T *)(uintptr_t)(v - r.sent[k] + r.real[k]);
}

int cache_mode() {   // 0 off, 1 on, 2 verify
    static const int mode = [] {
        const char *e = getenv("METALBLAS_LAUNCH_CACHE");
        if (!e) return 1;
        if (strcmp(e, "0") == 0) return 0;
        if (strcmp(e, "verify") == 0) return 2;
        return 1;
    }();
    return mode;
}

std::mutex g_cache_mu;
std::unordered_map<std::string, CallPlan> g_cache;
constexpr size_t kCacheCap = 1024;

static_assert(sizeof(mb_gemm_desc) == 296, "mb_gemm_desc has padding: the signature would read it");

// The cached plan of desc's signature, relocated to desc's operands, in cp.
int cached_plan(const mb_gemm_desc *desc, CallPlan &cp) {
    mb_gemm_desc canon = *desc;
    Reloc r;
    mb_matrix *ops[4] = {&canon.a, &canon.b, &canon.c, &canon.bias};
    for (int k = 0; k < 4; ++k) {
        const uint64_t real = (uint64_t)(uintptr_t)ops[k]->ptr;
        r.real[k] = real;
        r.sent[k] = real ? kSentBase + (uint64_t)k * kSentSpan + (real & 255) : 0;
        ops[k]->ptr = (void *)(uintptr_t)r.sent[k];
    }
    canon.workspace = (void *)(uintptr_t)(desc->workspace ? 1 : 0);
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::string key((const char *)&canon, sizeof(canon));
    key.append((const char *)&dev, sizeof(dev));
    bool hit = false;
    {
        std::lock_guard<std::mutex> lk(g_cache_mu);
        auto it = g_cache.find(key);
        if (it != g_cache.end()) {
            cp = it->second;
            hit = true;
        }
    }
    if (!hit) {
        const int st = plan_call(&canon, cp);
        if (st != MB_OK) return st;
        std::lock_guard<std::mutex> lk(g_cache_mu);
        if (g_cache.size() >= kCacheCap) g_cache.clear();
        g_cache.emplace(std::move(key), cp);
    }
    for (int i = 0; i < cp.n; ++i) each_ptr(cp.part[i], [&](auto *&p) { relocate(p, r); });
    for (int i = 0; i < cp.ncopy; ++i) relocate(cp.copy[i].a.src, r);
    if (hit && cache_mode() == 2) {
        CallPlan fresh;
        const int st = plan_call(desc, fresh);
        bool same = st == MB_OK && fresh.n == cp.n && fresh.ncopy == cp.ncopy && fresh.copy_bytes == cp.copy_bytes;
        for (int i = 0; same && i < cp.ncopy; ++i)
            same = fresh.copy[i].a.src == cp.copy[i].a.src && fresh.copy[i].off == cp.copy[i].off;
        for (int i = 0; same && i < cp.n; ++i) {
            Plan &x = cp.part[i], &y = fresh.part[i];
            uint64_t px[32], py[32];
            int nx = 0, ny = 0;
            each_ptr(x, [&](auto *&p) { px[nx++] = (uint64_t)(uintptr_t)p; });
            each_ptr(y, [&](auto *&p) { py[ny++] = (uint64_t)(uintptr_t)p; });
            for (int j = 0; j < nx && j < ny; ++j)
                if (px[j] != py[j])
                    fprintf(stderr, "metalblas_amd: part %d pointer field %d: relocated %llx, fresh %llx\n", i, j,
                            (unsigned long long)px[j], (unsigned long long)py[j]);
            same = nx == ny && memcmp(px, py, sizeof(uint64_t) * nx) == 0 && x.family == y.family &&
                   x.ws_bytes == y.ws_bytes && x.split_off == y.split_off && x.tile.bm == y.tile.bm &&
                   x.tile.bn == y.tile.bn && x.tile.sched == y.tile.sched && x.gg.splits == y.gg.splits &&
                   x.gg.k_chunk == y.gg.k_chunk && x.gv.splits == y.gv.splits && x.gemv_fast == y.gemv_fast &&
                   x.pack[0].on == y.pack[0].on && x.pack[1].on == y.pack[1].on && x.cplx == y.cplx &&
                   x.p.transposed == y.p.transposed && x.gen_bt == y.gen_bt;
        }
        if (!same) {
            fprintf(stderr, "metalblas_amd: relocated plan differs from a fresh plan (dtype %d, %lld x %lld x %lld)\n",
                    desc->dtype, (long long)desc->M, (long long)desc->N, (long long)desc->K);
            abort();
        }
    }
    return MB_OK;
}

// ---- allocation-free entry point -----------------------------------------------------------
// mb_gemm_noalloc runs on this file-scope device array instead of a caller's workspace.  Each
// device that loads the library holds its own copy (64 MiB) until the process ends.  In host
// code `scratch` is only a host-side stand-in for the symbol: its device address on the current
// device comes from hipGetSymbolAddress, taken once per device on the first call there and kept
// in g_scratch_ptr; only that address is ever handed to a kernel.  No byte of it needs to start
// at zero: every scratch byte a kernel reads (split-K partial planes, operand copies, the complex
// expansion) was written earlier in the same call.  Calls that overlap on one device (other
// streams, other host threads) share the array and race.
std::mutex g_scratch_mu;
void *g_scratch_ptr[64];

int scratch_address(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return MB_ERR_NO_DEVICE;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return MB_ERR_NO_DEVICE;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return MB_OK;
}

int gemm_impl(const mb_gemm_desc *desc, void *stream);

}  // namespace

extern "C" {

int mb_gemm(const mb_gemm_desc *desc, void *stream) {
    if (!desc) return MB_ERR_INVALID_ARG;
    if (internal_flags(desc)) return MB_ERR_INVALID_ARG;
    return gemm_impl(desc, stream);
}

int mb_gemm_noalloc(const mb_gemm_desc *desc, void *stream) {
    if (!desc) return MB_ERR_INVALID_ARG;
    if (desc->flags & ~MB_FLAG_DRY_RUN) return MB_ERR_INVALID_ARG;
    mb_gemm_desc d = *desc;
    void *p = nullptr;
    const int st = scratch_address(&p);
    if (st != MB_OK) return st;
    d.workspace = p;
    d.workspace_bytes = kScratchBytes;
    d.flags |= kFlagStaticScratch;
    return gemm_impl(&d, stream);
}

int64_t mb_gemm_noalloc_scratch_bytes(void) { return kScratchBytes; }

}  // extern "C"

namespace {

// a packed peel's sentinel pointer (spans 4..6) -> its place in the workspace copies
template <class T>
void place_copy(T *&ptr, const CallPlan &cp, char *wsb) {
    const uint64_t v = (uint64_t)(uintptr_t)ptr;
    if (v < kSentCopy || v >= kSentCopy + (uint64_t)cp.ncopy * kSentSpan) return;
    const int k = (int)((v - kSentCopy) / kSentSpan);
    ptr = (T *)(wsb + cp.copy[k].off + (v - kSentCopy - (uint64_t)k * kSentSpan));
}

int gemm_impl(const mb_gemm_desc *desc, void *stream) {
    CallPlan cp;
    const int st = cache_mode() ? cached_plan(desc, cp) : plan_call(desc, cp);
    if (st != MB_OK) return st;
    if (desc->flags & MB_FLAG_DRY_RUN) return MB_OK;
    if (cp.ncopy > 0) {
        // packed peel: the operand copies first, then the parts on them, each part's own
        // workspace after the copies
        if (!desc->workspace || desc->workspace_bytes < call_ws_bytes(cp)) return MB_ERR_WORKSPACE;
        char *wsb = (char *)desc->workspace;
        PackArgs a[3];
        for (int i = 0; i < cp.ncopy; ++i) {
            a[i] = cp.copy[i].a;
            a[i].dst = wsb + cp.copy[i].off;
        }
        int i = 0;
        if (cp.ncopy >= 2) {   // the copies of A and B in one launch
            if (launch_pack2(a[0], a[1], (hipStream_t)stream) != hipSuccess) return MB_ERR_LAUNCH;
            i = 2;
        }
        for (; i < cp.ncopy; ++i)
            if (launch_pack(a[i], (hipStream_t)stream) != hipSuccess) return MB_ERR_LAUNCH;
        mb_gemm_desc rest = *desc;
        rest.workspace = wsb + cp.copy_bytes;
        rest.workspace_bytes = desc->workspace_bytes - cp.copy_bytes;
        for (int i = 0; i < cp.n; ++i) {
            each_ptr(cp.part[i], [&](auto *&p) { place_copy(p, cp, wsb); });
            const int rs = run_plan(cp.part[i], &rest, (hipStream_t)stream, nullptr);
            if (rs != MB_OK) return rs;
        }
        return MB_OK;
    }
    // the parts of a peeled product run one after another on the caller's stream and share
    // its workspace (each part's descriptor is desc with offset operands)
    for (int i = 0; i < cp.n; ++i) {
        const int rs = run_plan(cp.part[i], desc, (hipStream_t)stream, nullptr);
        if (rs != MB_OK) return rs;
    }
    return MB_OK;
}

}  // namespace

extern "C" {

int64_t mb_gemm_workspace_bytes(const mb_gemm_desc *desc) {
    if (internal_flags(desc)) return MB_ERR_INVALID_ARG;
    Peel pe;
    if (desc && plan_peel(desc, pe)) {   // the parts run one after another: the largest need
        int64_t ws = 0;
        for (int i = 0; i < pe.n; ++i) {
            Plan pl;
            const int st = make_plan(&pe.part[i], pl);
            if (st != MB_OK) return st;
            ws = std::max<int64_t>(ws, pl.ws_bytes);
        }
        return ws;
    }
    CallPlan cp;
    if (desc && plan_packed_peel(desc, cp, true)) return call_ws_bytes(cp);
    Plan pl;
    int st = make_plan(desc, pl);
    if (st != MB_OK) return st;
    return pl.ws_bytes;
}

int mb_plan(const mb_gemm_desc *desc, mb_plan_info *info) {
    if (!info || internal_flags(desc)) return MB_ERR_INVALID_ARG;
    Plan pl;
    Peel pe;
    CallPlan cp;
    // a peeled product reports its core (the strips run on the GEMV / thin kernels)
    const bool peeled = desc && plan_peel(desc, pe);
    const bool packed_peel = !peeled && desc && plan_packed_peel(desc, cp, true);
    int st = MB_OK;
    if (packed_peel)
        pl = cp.part[0];
    else
        st = make_plan(peeled ? &pe.part[0] : desc, pl);
    if (st != MB_OK) return st;
    memset(info, 0, sizeof(*info));
    info->family = pl.family;
    info->transposed = pl.p.transposed;
    info->workspace_bytes = peeled || packed_peel ? mb_gemm_workspace_bytes(desc) : pl.ws_bytes;
    info->split_k = 1;
    if (pl.family == MB_FAMILY_MFMA) {
        info->tile[0] = pl.tile.bm;
        info->tile[1] = pl.tile.bn;
        info->tile[2] = 8 * (16 / dtype_size(pl.p.dt));
        info->tile[3] = pl.tile.wm;
        info->tile[4] = pl.tile.wn;
        info->tile[5] = pl.tile.sched + 1;
        info->tile[6] = pl.a_kc;
        info->tile[7] = pl.b_kc;
        info->split_k = pl.gg.splits;
        info->swizzle_log = pl.gg.swz;
        const bool dot4 = pl.tile.bm == 4 && pl.tile.bn == 16;   // k_thin_dot4: 256 threads, persistent
        const bool dotx = pl.tile.bm == 4 && pl.tile.bn == 8;    // k_dotx: one wave per 1024 of K
        info->block = dot4 ? 256 : dotx ? 64 * m16::dotx_waves(pl.p.K) : 64 * pl.tile.wm * pl.tile.wn;
        info->grid[0] = pl.gg.persist > 0 ? pl.gg.persist
                                          : (int)(((pl.p.M + pl.tile.bm - 1) / pl.tile.bm) * ((pl.p.N + pl.tile.bn - 1) / pl.tile.bn));
        info->grid[1] = pl.gg.splits;
        if (pl.tile.sched == 2) {   // deep-K: one 1-D grid of (K slice, tile) workgroups
            info->grid[0] *= pl.gg.splits;
            info->grid[1] = 1;
        }
        info->grid[2] = pl.gg.zblocks > 0 ? pl.gg.zblocks : (int)(pl.p.batch < 65535 ? pl.p.batch : 65535);
    } else if (pl.family == MB_FAMILY_GENERIC) {
        info->tile[0] = pl.gen_bt;
        info->tile[1] = pl.gen_bt;
        info->tile[2] = pl.gen_bt == 16 ? 128 : pl.gen_bt == 32 ? 64 : 16;
        info->split_k = pl.gg.splits;
        info->block = 256;
    } else if (pl.family == MB_FAMILY_GEMV_DOT || pl.family == MB_FAMILY_GEMV_AXPY) {
        info->tile[0] = pl.gv.nv;
        info->tile[1] = pl.gv.vec_ok;
        info->tile[2] = pl.gemv_fast;
        info->split_k = pl.gv.splits;
        info->block = 256;
    }
    return MB_OK;
}

int mb_tile_candidates(const mb_gemm_desc *desc, int32_t *tiles, int cap) {
    if (internal_flags(desc)) return MB_ERR_INVALID_ARG;
    Plan pl;
    int st = make_plan(desc, pl);
    if (st != MB_OK) return st;
    const bool mfma = pl.family == MB_FAMILY_MFMA;
    const bool gemv = pl.family == MB_FAMILY_GEMV_DOT || pl.family == MB_FAMILY_GEMV_AXPY;
    if (!mfma && !gemv) return 0;
    const int dt = desc->dtype;
    const int bk = 8 * (16 / dtype_size(dt));
    int out = 0;
    // plan identities already listed (family, tile, K slices): a request that plans like an
    // earlier entry is not listed again
    struct Ident {
        int family, bm, bn, wm, wn, sched, splits;
    };
    Ident seen[48];
    int nseen = 0;
    auto ident = [](const Plan &q) {
        const bool m = q.family == MB_FAMILY_MFMA;
        return Ident{q.family, m ? q.tile.bm : 0, m ? q.tile.bn : 0, m ? q.tile.wm : 0, m ? q.tile.wn : 0,
                     m ? q.tile.sched : 0, m ? q.gg.splits : q.gv.splits};
    };
    auto fresh = [&](const Ident &x) {
        for (int i = 0; i < nseen; ++i)
            if (!memcmp(&seen[i], &x, sizeof(Ident))) return false;
        if (nseen < 48) seen[nseen++] = x;
        return true;
    };
    auto put = [&](const MfmaTile &t, int split) {
        if (out < cap && tiles) {
            int32_t *q = tiles + 8 * out;
            memset(q, 0, 8 * sizeof(int32_t));
            if (t.bm > 0) {
                q[0] = t.bm; q[1] = t.bn; q[2] = bk; q[3] = t.wm; q[4] = t.wn; q[5] = t.sched + 1;
            }
            q[6] = split;
        }
        ++out;
    };
    // entry 0: the static plan (its matrix-core tile, or zeros for a GEMV plan); a tuner runs it
    // without a request (a tile request turns edge peeling off)
    {
        // an edge-peeled product runs the peel: entry 0 shows its core (as mb_plan does), and
        // every whole-product tile is a rival
        Peel pe;
        CallPlan cp;
        Plan core;
        if (plan_peel(desc, pe) && make_plan(&pe.part[0], core) == MB_OK) {
            put(core.tile, 0);
        } else if (plan_packed_peel(desc, cp, true)) {
            put(cp.part[0].tile, 0);
        } else {
            put(mfma ? pl.tile : MfmaTile{0, 0, 0, 0, 0}, 0);
            fresh(ident(pl));
        }
    }
    // a request: listed when it plans to the requested tile (and K slices) and differs from
    // every plan listed before
    auto offer = [&](const MfmaTile &t, int split) {
        if (out >= cap && tiles) return;
        mb_gemm_desc d = *desc;
        d.tile[0] = t.bm; d.tile[1] = t.bn; d.tile[2] = 0; d.tile[3] = t.wm; d.tile[4] = t.wn; d.tile[5] = t.sched + 1;
        d.tile[6] = d.tile[7] = 0;
        d.split_k = split;
        Plan q;
        if (make_plan(&d, q) != MB_OK || q.family != MB_FAMILY_MFMA) return;
        if (q.tile.bm != t.bm || q.tile.bn != t.bn || q.tile.sched != t.sched) return;
        if (split > 0 && q.gg.splits != split) return;
        if (fresh(ident(q))) put(t, split);
    };
    const Prob &p = pl.p;   // the planned problem (a column-major output is the transposed one)
    if (pl.cplx || !mfma_supported_dtype(dt)) return out;
    MfmaTile list[32];
    const int n = mfma_list_tiles(dt, list, 32);
    const bool f16 = dt == MB_DTYPE_BF16 || dt == MB_DTYPE_F16;
    // (a) the thin-product kernels, for a bf16 / fp16 product with at most 32 rows or columns
    //     (the reference times its gemv_bt / flipt / sgpipe kernels against the tiles,
    //     metalblas/float_dispatch.py:439-481, 516-542)
    if (f16 && (desc->M <= 32 || desc->N <= 32)) {
        static const MfmaTile thin[] = {{4, 8, m16::kDotxMaxWaves, 1, 0}, {4, 16, 1, 1, 0}, {64, 16, 4, 1, 0},
                                        {32, 128, 1, 4, 0}, {32, 256, 1, 4, 0}};
        for (const MfmaTile &t : thin) offer(t, 0);
    }
    // (b) the tile family (matrix-core tiles other than the thin and deep-K schedules), for
    //     products that are not a single vector.  When the static tile already gives every CU
    //     two tiles over a K of at least 1024, tiles of less than a quarter of its area are not
    //     offered: they load more bytes per flop and cannot win there, and timing them (the
    //     32 x 32 register-staged tile takes tens of milliseconds at 8192^3) only delays the
    //     first call and heats the board before the work that follows.  Over a short K the
    //     small tiles stay (chained batch entries on them beat the large tiles: bf16 bmm
    //     192 x 512 x 512 x 64, 64 x 128 32.8 us against 35.2 us on 256 x 256)
    if (desc->M > 1 && desc->N > 1) {
        const int64_t static_tiles =
            mfma ? ((p.M + pl.tile.bm - 1) / pl.tile.bm) * ((p.N + pl.tile.bn - 1) / pl.tile.bn) * p.batch : 0;
        const bool plenty = static_tiles >= 2LL * dev_info().cus && p.K >= 1024;
        for (int i = 0; i < n && i < 32; ++i) {
            const MfmaTile &t = list[i];
            if (thin_tile(t) || t.sched == 2) continue;
            if (t.bm > 2 * p.M + 32 || t.bn > 2 * p.N + 32) continue;
            if (plenty && 4LL * t.bm * t.bn < (int64_t)pl.tile.bm * pl.tile.bn) continue;
            offer(t, 0);
        }
    }
    // (c) K slices of the static tile: one slice more coarsely or finely split than the
    //     planner's choice (the reference's split-K candidates, float_dispatch.py:439-481);
    //     the deep-K schedule halves or doubles its slice count (unsplit, its few tiles would
    //     leave almost every CU idle)
    if (mfma && !thin_tile(pl.tile) && p.K >= 2048) {
        const int s = pl.gg.splits;
        const bool deep = pl.tile.sched == 2;
        for (int v : {s > 1 ? s / 2 : 0, s > 1 && !deep ? 1 : 0, 2 * s})
            if (v >= 1 && v != s && v <= (deep ? 128 : 64) && p.K / v >= 4 * bk) offer(pl.tile, v);
    }
    return out < cap ? out : cap;
}

int64_t mb_query(int32_t what) {
    switch (what) {
        case MB_QUERY_ABI_VERSION: return MB_ABI_VERSION;
        case MB_QUERY_HAS_MATRIX_CORES: return dev_info().arch == 950 ? 1 : 0;
        case MB_QUERY_CU_COUNT: return dev_info().cus;
        case MB_QUERY_GFX_ARCH: return dev_info().arch;
        case MB_QUERY_LDS_BYTES: return dev_info().lds;
    }
    return MB_ERR_INVALID_ARG;
}

const char *mb_strerror(int32_t status) {
    switch (status) {
        case MB_OK: return "success";
        case MB_ERR_INVALID_ARG: return "invalid argument";
        case MB_ERR_UNSUPPORTED_DTYPE: return "unsupported dtype";
        case MB_ERR_UNSUPPORTED_LAYOUT: return "unsupported layout for the requested backend";
        case MB_ERR_WORKSPACE: return "workspace missing or too small";
        case MB_ERR_LAUNCH: return "kernel launch failed";
        case MB_ERR_NO_DEVICE: return "no HIP device";
        case MB_ERR_GEMV_SHAPE: return "gemv backend requires M==1 or N==1";
        case MB_ERR_BAD_BACKEND: return "unknown backend";
        case MB_ERR_SCRATCH_LIMIT:
            return "the product needs more scratch than mb_gemm_noalloc's static buffer holds "
                   "(mb_gemm_noalloc_scratch_bytes()); call mb_gemm with a workspace instead";
    }
    return "unknown status";
}

}  // extern "C"
