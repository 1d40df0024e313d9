// Matrix-core GEMM instantiations for f16_t.
#include "mfma_gemm.hpp"

namespace mb {
namespace mfma {
hipError_t launch_f16(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    return launch_typed<f16_t>(t, a_kc, b_kc, g, grid, st);
}
}  // namespace mfma
}  // namespace mb
