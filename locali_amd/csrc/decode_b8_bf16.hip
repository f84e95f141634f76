// Decode kernels instantiated for 8-bit codes with bf16 activations.
#include "decode_kernels.hpp"

namespace locali {

hipError_t decode_b8_bf16(int which, int gpc, int cpr, const DecodeLaunch &L, hipStream_t st) {
    if (gpc != 1) return hipErrorInvalidValue;
    return decode_geometry<8, true, 1>(which, cpr, L, st);
}

}  // namespace locali
