// Matrix-core decode gate/up kernel instantiated for 2-bit codes (bf16 and
// fp16 activations).
#include "mfma_decode.hpp"

namespace locali {

hipError_t decode_diag_b2(const DecodeLaunch &L, hipStream_t st) {
    return L.bf16 ? launch_gateup_diag<2, true>(L, st) : launch_gateup_diag<2, false>(L, st);
}

}  // namespace locali
