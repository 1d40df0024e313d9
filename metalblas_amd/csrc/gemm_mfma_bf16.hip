// Matrix-core GEMM instantiations for bf16_t.
#include "mfma_gemm.hpp"

namespace mb {
namespace mfma {
hipError_t launch_bf16(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    return launch_typed<bf16_t>(t, a_kc, b_kc, g, grid, st);
}
}  // namespace mfma
}  // namespace mb
