// MFMA grouped kernels instantiated for 3-bit codes: the 4-bit kernels (input
// preparation, 64-position tiles) reading 3-bit rows and widening each lane's
// 32 values to 4-bit codes as they are consumed (bf16 and fp16 activations).
// Tiles of every size take the 64-position kernels: there are no small-tile
// kernels for 3-bit codes.
#include "mfma_wide.hpp"

namespace locali {

hipError_t mfma_b3(int which, bool bf16, const MfmaLaunch &L, hipStream_t st) {
    if (which == 5) return bf16 ? launch_place_prep<4, true>(L, st) : launch_place_prep<4, false>(L, st);
    if (which == 1 || which == 2)
        return bf16 ? launch_wide_stage<4, true, 3>(which, L, st) : launch_wide_stage<4, false, 3>(which, L, st);
    if (which == 0) return bf16 ? launch_mfma_prep<4, true>(L, st) : launch_mfma_prep<4, false>(L, st);
    return hipErrorInvalidValue;
}

}  // namespace locali
