// Grouped kernels instantiated for 8-bit codes with bf16 activations.
#include "grouped_kernels.hpp"

namespace locali {

hipError_t grouped_b8_bf16(int which, int gpc, int cpr, const GroupedKernelLaunch &L,
                           hipStream_t st) {
    if (gpc != 1) return hipErrorInvalidValue;
    return grouped_geometry<8, true, 1>(which, cpr, L, st);
}

}  // namespace locali
