// Grouped kernels instantiated for 2-bit codes with bf16 activations
// (one group per 16-byte chunk: group size >= 64).
#include "grouped_kernels.hpp"

namespace locali {

hipError_t grouped_b2g32_bf16(int which, int cpr, const GroupedKernelLaunch &L, hipStream_t st);

hipError_t grouped_b2_bf16(int which, int gpc, int cpr, const GroupedKernelLaunch &L, hipStream_t st) {
    if (gpc == 2) return grouped_b2g32_bf16(which, cpr, L, st);
    return grouped_geometry<2, true, 1>(which, cpr, L, st);
}

}  // namespace locali
