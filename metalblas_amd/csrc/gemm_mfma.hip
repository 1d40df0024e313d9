// Matrix-core GEMM family: compiled tile table and dtype dispatch.  The kernel template lives
// in mfma_gemm.hpp; each dtype is instantiated in its own translation unit
// (gemm_mfma_<dtype>.hip) so the build compiles them in parallel.
#include "launch.hpp"

namespace mb {

namespace mfma {
hipError_t launch_bf16(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_f16(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_f32(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_i8(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_u8(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
}  // namespace mfma
namespace m16 {
hipError_t launch_bf16_kwhole(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_bf16_ktail(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_f16_kwhole(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_f16_ktail(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_bf16_pp(bool ktail, int bn, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_f16_pp(bool ktail, int bn, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_i8_kwhole(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_i8_ktail(const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_i8_pp(bool ktail, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_thin(int dt, bool ktail, const MfmaTile &, bool, bool, const GemmArgs &, dim3, hipStream_t);
hipError_t launch_deepk(int dt, bool ktail, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st);
}  // namespace m16

namespace {
// ---- compiled tile table ----------------------------------------------------------------
struct TileEntry {
    int bm, bn, wm, wn, sched;
};
// register-staged family (mfma_gemm.hpp): every matrix-core dtype
constexpr TileEntry kTiles[] = {
    {256, 256, 2, 2, 0}, {256, 128, 2, 2, 0}, {128, 256, 2, 2, 0}, {128, 128, 2, 2, 0},
    {128, 64, 2, 2, 0},  {64, 128, 2, 2, 0},  {64, 64, 2, 2, 0},   {32, 32, 1, 1, 0},
};
// LDS-direct family (mfma16.hpp): bf16 / fp16 / int8 / uint8; sched 1 = the ping-pong kernel
// (256 x 128 ping-pong: bf16 / fp16 only)
constexpr TileEntry kTiles16[] = {
    {256, 256, 2, 4, 1}, {256, 128, 2, 4, 1}, {256, 256, 2, 2, 0}, {256, 256, 2, 4, 0}, {256, 128, 2, 2, 0}, {128, 256, 2, 2, 0},
    {128, 128, 2, 2, 0}, {128, 64, 2, 2, 0},  {64, 128, 2, 2, 0},  {64, 64, 2, 2, 0},  {32, 32, 1, 1, 0},
    // thin tiles for products with a few vectors (bf16 / fp16): k_thin_dot 64 x 16 and
    // k_thin_dot4 4 x 16 (A and B K-contiguous), k_thin16 32 x 256 and 32 x 128 (A
    // K-contiguous, B N-contiguous), k_dotx 4 x 8 (A K-contiguous, up to 16 waves over the
    // whole K)
    {64, 16, 4, 1, 0},   {32, 256, 1, 4, 0},  {32, 128, 1, 4, 0}, {4, 16, 1, 1, 0},  {4, 8, 16, 1, 0},
    // the deep-K schedule of the 64 x 64 tile (bf16 / fp16): few output tiles, many K slices
    {64, 64, 2, 2, 2},
};

// dtypes of the LDS-direct family
bool is16(int dt) { return dt == BF16 || dt == F16 || dt == I8 || dt == U8; }

bool in_table(const TileEntry *tb, int n, const MfmaTile &t) {
    for (int i = 0; i < n; ++i)
        if (tb[i].bm == t.bm && tb[i].bn == t.bn && tb[i].wm == t.wm && tb[i].wn == t.wn && tb[i].sched == t.sched)
            return true;
    return false;
}

// The LDS-direct loads address each operand tile with 31-bit byte offsets from the tile's
// first element; larger spans take the register-staged kernel.
bool m16_offsets_fit(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, int es) {
    const int64_t lim = (int64_t)1 << 30;
    const int64_t lda = a_kc ? g.a_rs : g.a_cs, ldb = b_kc ? g.b_cs : g.b_rs;
    const int64_t K = (int64_t)g.k_chunk + 128 / es;
    const int64_t ea = a_kc ? (int64_t)t.bm * lda + K : K * lda + t.bm;
    const int64_t eb = b_kc ? (int64_t)t.bn * ldb + K : K * ldb + t.bn;
    return ea * es < lim && eb * es < lim;
}

}  // namespace

bool mfma_supported_dtype(int dt) { return dt == BF16 || dt == F16 || dt == F32 || dt == I8 || dt == U8; }

int mfma_k_align(int dt) { return 16 / dtype_size(dt); }

bool mfma_tile_compiled(int dt, const MfmaTile &t) {
    if ((dt == I8 || dt == U8) && t.sched == 1 && t.bn != 256) return false;   // 8-bit ping-pong: 256 x 256 only
    if (t.sched == 2 && dt != BF16 && dt != F16) return false;                  // deep-K: 16-bit floats only
    if (is16(dt)) return in_table(kTiles16, sizeof(kTiles16) / sizeof(kTiles16[0]), t);
    return in_table(kTiles, sizeof(kTiles) / sizeof(kTiles[0]), t);
}

int mfma_list_tiles(int dt, MfmaTile *out, int cap) {
    const TileEntry *tb = is16(dt) ? kTiles16 : kTiles;
    const int cnt = is16(dt) ? (int)(sizeof(kTiles16) / sizeof(kTiles16[0])) : (int)(sizeof(kTiles) / sizeof(kTiles[0]));
    int n = 0;
    for (int i = 0; i < cnt; ++i) {
        const MfmaTile t{tb[i].bm, tb[i].bn, tb[i].wm, tb[i].wn, tb[i].sched};
        if (!mfma_tile_compiled(dt, t)) continue;   // e.g. the 8-bit ping-pong exists at 256 x 256 only
        if (n < cap) out[n] = t;
        ++n;
    }
    return n;
}

hipError_t launch_mfma(int dt, const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, hipStream_t st,
                       LaunchShape *shape) {
    const int tiles = cdiv(g.M, t.bm) * cdiv(g.N, t.bn);
    dim3 grid(g.persist > 0 ? g.persist : tiles, g.splits, g.zblocks > 0 ? g.zblocks : g.batch < 65535 ? g.batch : 65535);
    const bool dotx = t.bm == 4 && t.bn == 8;   // k_dotx: one wave per 1024 of K
    if (shape) *shape = {grid, dim3(t.bm == 4 && t.bn == 16 ? 256 : dotx ? 64 * m16::dotx_waves(g.K) : 64 * t.wm * t.wn)};
    if (is16(dt) && !(t.bm == 32 && t.bn == 32)) {
        const int es = dtype_size(dt), bk = 128 / es;
        if (m16_offsets_fit(t, a_kc, b_kc, g, es)) {
            const bool whole = (g.k_chunk % bk) == 0 && (g.K % bk) == 0;
            if ((t.bm == 64 && t.bn == 16) || (t.bm == 32 && (t.bn == 256 || t.bn == 128)) || (t.bm == 4 && t.bn == 16) ||
                dotx)
                return m16::launch_thin(dt, !whole, t, a_kc, b_kc, g, grid, st);
            if (t.sched == 2) {   // deep-K: a 1-D grid of (K slice, tile) workgroups
                const dim3 g1(tiles * g.splits, 1, grid.z);
                if (shape) *shape = {g1, dim3(256)};
                return m16::launch_deepk(dt, !whole, a_kc, b_kc, g, g1, st);
            }
            if (t.sched == 1) {
                if (dt == BF16) return m16::launch_bf16_pp(!whole, t.bn, a_kc, b_kc, g, grid, st);
                if (dt == F16) return m16::launch_f16_pp(!whole, t.bn, a_kc, b_kc, g, grid, st);
                if (t.bn != 256) return hipErrorInvalidValue;
                return m16::launch_i8_pp(!whole, a_kc, b_kc, g, grid, st);   // int8 and uint8
            }
            if (dt == BF16)
                return whole ? m16::launch_bf16_kwhole(t, a_kc, b_kc, g, grid, st)
                             : m16::launch_bf16_ktail(t, a_kc, b_kc, g, grid, st);
            if (dt == F16)
                return whole ? m16::launch_f16_kwhole(t, a_kc, b_kc, g, grid, st)
                             : m16::launch_f16_ktail(t, a_kc, b_kc, g, grid, st);
            return whole ? m16::launch_i8_kwhole(t, a_kc, b_kc, g, grid, st)
                         : m16::launch_i8_ktail(t, a_kc, b_kc, g, grid, st);
        }
        // very large leading dimensions: register-staged kernel with a compiled 4-wave tile
        MfmaTile v = in_table(kTiles, sizeof(kTiles) / sizeof(kTiles[0]), t) ? t : MfmaTile{128, 128, 2, 2, 0};
        dim3 grid2(cdiv(g.M, v.bm) * cdiv(g.N, v.bn), g.splits, grid.z);
        if (shape) *shape = {grid2, dim3(64 * v.wm * v.wn)};
        switch (dt) {
            case BF16: return mfma::launch_bf16(v, a_kc, b_kc, g, grid2, st);
            case F16: return mfma::launch_f16(v, a_kc, b_kc, g, grid2, st);
            case I8: return mfma::launch_i8(v, a_kc, b_kc, g, grid2, st);
            default: return mfma::launch_u8(v, a_kc, b_kc, g, grid2, st);
        }
    }
    switch (dt) {
        case BF16: return mfma::launch_bf16(t, a_kc, b_kc, g, grid, st);
        case F16: return mfma::launch_f16(t, a_kc, b_kc, g, grid, st);
        case F32: return mfma::launch_f32(t, a_kc, b_kc, g, grid, st);
        case I8: return mfma::launch_i8(t, a_kc, b_kc, g, grid, st);
        case U8: return mfma::launch_u8(t, a_kc, b_kc, g, grid, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace mb
