// Decode kernels for 3-bit codes with f16 activations: the 4-bit kernels
// reading 3-bit rows (each 32-value chunk widened to 4-bit codes on load).
#include "decode_kernels.hpp"

namespace locali {

hipError_t decode_b3_f16(int which, int gpc, int cpr, const DecodeLaunch &L, hipStream_t st) {
    if (gpc != 1) return hipErrorInvalidValue;
    return decode_geometry<4, false, 1, 3>(which, cpr, L, st);
}

}  // namespace locali
