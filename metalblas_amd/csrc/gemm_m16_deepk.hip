// Deep-K schedule instantiations (bf16_t / f16_t): k_thin16 on 64 x 64 tiles over a 1-D grid of
// (K slice, tile) workgroups in slice_coords order (mfma16.hpp).
#include "mfma16.hpp"

namespace mb {
namespace m16 {
hipError_t launch_deepk(int dt, bool ktail, bool a_kc, bool b_kc, const GemmArgs &g, dim3 grid, hipStream_t st) {
    if (dt == BF16)
        return ktail ? launch_deepk16<bf16_t, true>(a_kc, b_kc, g, grid, st)
                     : launch_deepk16<bf16_t, false>(a_kc, b_kc, g, grid, st);
    if (dt == F16)
        return ktail ? launch_deepk16<f16_t, true>(a_kc, b_kc, g, grid, st)
                     : launch_deepk16<f16_t, false>(a_kc, b_kc, g, grid, st);
    return hipErrorInvalidValue;
}
}  // namespace m16
}  // namespace mb
