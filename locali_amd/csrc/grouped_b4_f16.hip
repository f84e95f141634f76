// Grouped kernels instantiated for 4-bit codes with f16 activations.
#include "grouped_kernels.hpp"

namespace locali {

hipError_t grouped_b4_f16(int which, int gpc, int cpr, const GroupedKernelLaunch &L,
                           hipStream_t st) {
    if (gpc != 1) return hipErrorInvalidValue;
    return grouped_geometry<4, false, 1>(which, cpr, L, st);
}

}  // namespace locali
