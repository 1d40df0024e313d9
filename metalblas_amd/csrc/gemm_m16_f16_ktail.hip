// LDS-direct matrix-core GEMM instantiations for f16_t, K slices ending inside a stage (kernel template in mfma16.hpp).
#include "mfma16.hpp"

namespace mb {
namespace m16 {
hipError_t launch_f16_ktail(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    return launch16_typed<f16_t, true>(t, a_kc, b_kc, g, grid, st);
}
}  // namespace m16
}  // namespace mb
