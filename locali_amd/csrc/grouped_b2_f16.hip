// Grouped kernels instantiated for 2-bit codes with f16 activations.
#include "grouped_kernels.hpp"

namespace locali {

hipError_t grouped_b2_f16(int which, int gpc, int cpr, const GroupedKernelLaunch &L,
                           hipStream_t st) {
    if (gpc == 2) return grouped_geometry<2, false, 2>(which, cpr, L, st);
    return grouped_geometry<2, false, 1>(which, cpr, L, st);
}

}  // namespace locali
