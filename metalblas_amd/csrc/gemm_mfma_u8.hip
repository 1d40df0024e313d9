// Matrix-core GEMM instantiations for uint8_t.
#include "mfma_gemm.hpp"

namespace mb {
namespace mfma {
hipError_t launch_u8(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    return launch_typed<uint8_t>(t, a_kc, b_kc, g, grid, st);
}
}  // namespace mfma
}  // namespace mb
