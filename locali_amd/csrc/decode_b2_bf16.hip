// Decode kernels instantiated for 2-bit codes with bf16 activations
// (one group per 16-byte chunk: group size >= 64).
#include "decode_kernels.hpp"

namespace locali {

hipError_t decode_b2g32_bf16(int which, int cpr, const DecodeLaunch &L, hipStream_t st);

hipError_t decode_b2_bf16(int which, int gpc, int cpr, const DecodeLaunch &L, hipStream_t st) {
    if (gpc == 2) return decode_b2g32_bf16(which, cpr, L, st);
    return decode_geometry<2, true, 1>(which, cpr, L, st);
}

}  // namespace locali
