// Decode kernels instantiated for 4-bit codes with f16 activations.
#include "decode_kernels.hpp"

namespace locali {

hipError_t decode_b4_f16(int which, int gpc, int cpr, const DecodeLaunch &L, hipStream_t st) {
    if (gpc != 1) return hipErrorInvalidValue;
    return decode_geometry<4, false, 1>(which, cpr, L, st);
}

}  // namespace locali
