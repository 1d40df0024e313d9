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

namespace {
// ---- compiled tile table ----------------------------------------------------------------
struct TileEntry {
    int bm, bn, wm, wn;
};
constexpr TileEntry kTiles[] = {
    {256, 256, 2, 2}, {256, 128, 2, 2}, {128, 256, 2, 2}, {128, 128, 2, 2},
    {128, 64, 2, 2},  {64, 128, 2, 2},  {64, 64, 2, 2},   {32, 32, 1, 1},
};

}  // namespace

bool mfma_supported_dtype(int dt) { return dt == BF16 || dt == F16 || dt == F32 || dt == I8 || dt == U8; }

int mfma_k_align(int dt) { return 16 / dtype_size(dt); }

bool mfma_tile_compiled(int, const MfmaTile &t) {
    for (const auto &e : kTiles)
        if (e.bm == t.bm && e.bn == t.bn && e.wm == t.wm && e.wn == t.wn) return true;
    return false;
}

int mfma_list_tiles(int, MfmaTile *out, int cap) {
    int n = 0;
    for (const auto &e : kTiles) {
        if (n < cap) out[n] = {e.bm, e.bn, e.wm, e.wn};
        ++n;
    }
    return n;
}

hipError_t launch_mfma(int dt, const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, hipStream_t st,
                       LaunchShape *shape) {
    const int tiles = cdiv(g.M, t.bm) * cdiv(g.N, t.bn);
    dim3 grid(tiles, g.splits, g.batch < 65535 ? g.batch : 65535);
    if (shape) *shape = {grid, dim3(64 * t.wm * t.wn)};
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
