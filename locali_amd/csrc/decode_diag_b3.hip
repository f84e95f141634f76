// Matrix-core decode gate/up kernel instantiated for 3-bit codes (bf16 and
// fp16 activations): the 4-bit kernel reading 12-byte pieces of the 3-bit
// rows and widening them to 4-bit codes as they arrive.
#include "mfma_decode.hpp"

namespace locali {

hipError_t decode_diag_b3(const DecodeLaunch &L, hipStream_t st) {
    return L.bf16 ? launch_gateup_diag<3, true>(L, st) : launch_gateup_diag<3, false>(L, st);
}

}  // namespace locali
