// Ping-pong LDS-direct matrix-core GEMM instantiations for int8 and uint8 (kernel template in
// mfma16.hpp).
#include "mfma16.hpp"

namespace mb {
namespace m16 {
hipError_t launch_i8_pp(bool ktail, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    return ktail ? launch16pp<int8_t, true>(a_kc, b_kc, g, grid, st) : launch16pp<int8_t, false>(a_kc, b_kc, g, grid, st);
}
}  // namespace m16
}  // namespace mb
