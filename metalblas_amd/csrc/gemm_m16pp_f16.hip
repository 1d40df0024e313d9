// Ping-pong LDS-direct matrix-core GEMM instantiations for f16_t (kernel template in mfma16.hpp).
#include "mfma16.hpp"

namespace mb {
namespace m16 {
hipError_t launch_f16_pp(bool ktail, int bn, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    if (bn == 128)
        return ktail ? launch16pp<f16_t, true, 128>(a_kc, b_kc, g, grid, st)
                     : launch16pp<f16_t, false, 128>(a_kc, b_kc, g, grid, st);
    return ktail ? launch16pp<f16_t, true>(a_kc, b_kc, g, grid, st) : launch16pp<f16_t, false>(a_kc, b_kc, g, grid, st);
}
}  // namespace m16
}  // namespace mb
