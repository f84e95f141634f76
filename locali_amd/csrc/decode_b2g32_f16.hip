// Decode kernels instantiated for 2-bit codes with f16 activations and
// group size 32 (two groups per 16-byte chunk).
#include "decode_kernels.hpp"

namespace locali {

hipError_t decode_b2g32_f16(int which, int cpr, const DecodeLaunch &L, hipStream_t st) {
    return decode_geometry<2, false, 2>(which, cpr, L, st);
}

}  // namespace locali
