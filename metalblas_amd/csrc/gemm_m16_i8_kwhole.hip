// LDS-direct matrix-core GEMM instantiations for int8 (and uint8, which shares the signed
// instruction and the truncating store), K slices made of whole stages (kernel template in mfma16.hpp).
#include "mfma16.hpp"

namespace mb {
namespace m16 {
hipError_t launch_i8_kwhole(const MfmaTile &t, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    return launch16_typed<int8_t, false>(t, a_kc, b_kc, g, grid, st);
}
}  // namespace m16
}  // namespace mb
