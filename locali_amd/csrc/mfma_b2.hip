// MFMA grouped kernels (16-position and small tiles) instantiated for 2-bit codes
// (bf16 and fp16 activations).
#include "mfma_small.hpp"

namespace locali {

hipError_t mfma_b2(int which, bool bf16, const MfmaLaunch &L, hipStream_t st) {
    if (which >= 3) return bf16 ? launch_small_stage<2, true>(which, L, st) : launch_small_stage<2, false>(which, L, st);
    return bf16 ? launch_mfma_stage<2, true>(which, L, st) : launch_mfma_stage<2, false>(which, L, st);
}

}  // namespace locali
