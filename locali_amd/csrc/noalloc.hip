// locali_moe_forward_noalloc: the whole-layer forward for callers that cannot
// allocate (code under HIP graph capture, tight serving loops). Its scratch is
// the file-scope device array below instead of a caller workspace: one copy
// per GPU, set up on the first call on each device and kept until the process
// ends. Every call on a GPU shares that GPU's copy, so calls that overlap on
// one GPU (different streams, different threads) race; serialise them.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "locali_moe.h"

namespace locali {
int set_error(int code, const char *msg);
// Keeps the grouped path's kernels on the caller's stream (no second stream
// or events are created) for the calling thread while set.
void set_no_alloc_call(bool on);
}

namespace {

constexpr size_t kScratchBytes = LOCALI_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Device address of each GPU's copy of `scratch` (nullptr until set up). In
// host code `scratch` names a host-side stand-in, never the device memory:
// only these addresses are passed to kernels.
void *g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

__global__ __launch_bounds__(256) void clear_scratch_kernel(uint4 *p, size_t n) {
    for (size_t i = blockIdx.x * size_t{256} + threadIdx.x; i < n; i += size_t{gridDim.x} * 256)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

int fail_hip(hipError_t e, const char *where) {
    char buf[256];
    snprintf(buf, sizeof(buf), "forward_noalloc: %s: %s", where, hipGetErrorString(e));
    return locali::set_error(LOCALI_E_HIP, buf);
}

// This GPU's scratch address; on the first call on a device, looks it up and
// clears it (a fill kernel on the caller's stream, ordered before the call's
// own kernels, which also records cleanly into a graph under capture).
int scratch_of_current_device(void **out, hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail_hip(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return locali::set_error(LOCALI_E_ARG, "forward_noalloc: device id too large");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return fail_hip(e, "hipGetSymbolAddress(scratch)");
        hipLaunchKernelGGL(clear_scratch_kernel, dim3(1024), dim3(256), 0, st, static_cast<uint4 *>(p),
                           kScratchBytes / sizeof(uint4));
        if ((e = hipGetLastError()) != hipSuccess) return fail_hip(e, "scratch clear launch");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return 0;
}

}  // namespace

extern "C" int locali_moe_forward_noalloc(const locali_router *router, const locali_expert_arena *routed,
                                          const locali_expert_arena *shared, const int32_t *slot_of_expert,
                                          const void *x, int32_t x_dtype, int32_t tokens,
                                          const int32_t *input_ids, float swiglu_limit, int32_t fp32_swiglu,
                                          void *out, int32_t *idx, float *weights, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    if (!router || !routed || tokens < 0)
        return locali::set_error(LOCALI_E_ARG, "forward_noalloc: bad arguments");
    const size_t need = locali_moe_workspace_bytes(tokens, routed->gate.cols, routed->gate.rows,
                                                   router->n_experts, router->top_k, shared ? 1 : 0);
    if (need == 0) return locali::set_error(LOCALI_E_ARG, "forward_noalloc: bad shapes");
    if (need > kScratchBytes) {
        char buf[256];
        snprintf(buf, sizeof(buf),
                 "forward_noalloc: %d tokens need %zu bytes of scratch; the static scratch holds %zu "
                 "(use locali_moe_forward with a workspace)", tokens, need, kScratchBytes);
        return locali::set_error(LOCALI_E_WORKSPACE, buf);
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    void *ws = nullptr;
    if (const int rc = scratch_of_current_device(&ws, st)) return rc;
    locali::set_no_alloc_call(true);
    const int rc = locali_moe_forward(router, routed, shared, slot_of_expert, x, x_dtype, tokens, input_ids,
                                      swiglu_limit, fp32_swiglu, out, idx, weights, ws, kScratchBytes, stream);
    locali::set_no_alloc_call(false);
    return rc;
}
