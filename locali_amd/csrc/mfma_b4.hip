// MFMA grouped kernels instantiated for 4-bit codes (bf16 and fp16 activations).
#include "mfma_grouped.hpp"

namespace locali {

hipError_t mfma_b4(int which, bool bf16, const MfmaLaunch &L, hipStream_t st) {
    return bf16 ? launch_mfma_stage<4, true>(which, L, st) : launch_mfma_stage<4, false>(which, L, st);
}

}  // namespace locali
