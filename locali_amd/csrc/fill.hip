// Batched arena fills: the records of one or more expert slots copied from
// pinned host memory into their arena regions by one kernel that reads the
// host memory over PCIe itself (the slot fills of arena.py:179-200 and
// ArenaStore._fill, one launch per call instead of one copy per record).
//
// The pieces travel in the kernel arguments; the host side gives each piece
// a run of consecutive workgroups, and every thread moves kFillUnits 16-byte
// units: all loads first (many PCIe reads in flight per wave), then the
// stores.
#include "launch.hpp"

namespace locali {

constexpr int kFillThreads = 256;
constexpr int kFillUnits = 8;   // 16-byte units per thread

__global__ __launch_bounds__(kFillThreads) void fill_kernel(FillBatch b) {
    // the piece owning this workgroup (uniform): last k with first_block[k] <= x
    int k = 0;
    for (int i = 1; i < b.n; ++i)
        if (b.first_block[i] <= static_cast<int>(blockIdx.x)) k = i;
    const u32x4 *src = reinterpret_cast<const u32x4 *>(b.src[k]);
    u32x4 *dst = reinterpret_cast<u32x4 *>(b.dst[k]);
    const int64_t units = b.units[k];
    const int64_t base = (static_cast<int64_t>(blockIdx.x) - b.first_block[k]) * (kFillThreads * kFillUnits) +
                         threadIdx.x;
    u32x4 v[kFillUnits];
#pragma unroll
    for (int i = 0; i < kFillUnits; ++i) {
        const int64_t u = base + static_cast<int64_t>(i) * kFillThreads;
        if (u < units) v[i] = __builtin_nontemporal_load(src + u);
    }
#pragma unroll
    for (int i = 0; i < kFillUnits; ++i) {
        const int64_t u = base + static_cast<int64_t>(i) * kFillThreads;
        if (u < units) dst[u] = v[i];
    }
}

hipError_t launch_fill(const FillBatch &b, int blocks, hipStream_t st) {
    hipLaunchKernelGGL(fill_kernel, dim3(blocks), dim3(kFillThreads), 0, st, b);
    return hipGetLastError();
}

int fill_blocks(int64_t units) {
    const int64_t per = kFillThreads * kFillUnits;
    return static_cast<int>((units + per - 1) / per);
}

}  // namespace locali
