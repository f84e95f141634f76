// MFMA grouped kernels (input preparation, 64-position and small tiles) instantiated for 2-bit codes
// (bf16 and fp16 activations).
#include "mfma_small.hpp"
#include "mfma_wide.hpp"

namespace locali {

hipError_t mfma_b2(int which, bool bf16, const MfmaLaunch &L, hipStream_t st) {
    if (which == 5) return bf16 ? launch_place_prep<2, true>(L, st) : launch_place_prep<2, false>(L, st);
    if (which == 3 || which == 4) return bf16 ? launch_small_stage<2, true>(which, L, st) : launch_small_stage<2, false>(which, L, st);
    if (which == 1 || which == 2) return bf16 ? launch_wide_stage<2, true>(which, L, st) : launch_wide_stage<2, false>(which, L, st);
    return bf16 ? launch_mfma_prep<2, true>(L, st) : launch_mfma_prep<2, false>(L, st);
}

}  // namespace locali
