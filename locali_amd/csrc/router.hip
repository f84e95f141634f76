// Router: logits = x . Wg^T (fp32 accumulate), score = f(logits), top-k on
// score + selection-only bias, weights renormalised and scaled.
//
// Semantics follow the DeepSeek-V4 gate the reference module delegates to
// (dsv4_arena.py:147-153, 165-166): sqrt(softplus) scores, e_score_correction
// bias used for selection only, weights = score[idx] / (sum + 1e-20) times
// routed_scaling_factor, hash routing idx = tid2eid[input_id] in hash layers;
// and Locali's own sigmoid router (arena.py:501-506). In-row order is
// canonical: descending selection value, ties to the lower expert id.
//
// Kernels
//   router_gemv_fast_kernel  decode (few tokens), gate and x of one 16-bit
//                        type, d = 512 * NCH: one wave per expert, all of a
//                        lane's 16-byte gate chunks and x chunks issued before
//                        the first v_dot2.
//   router_gemv_kernel   the same for any gate dtype and d % 8 == 0.
//   router_mfma_kernel   prefill: 32 tokens x 32 experts per wave with
//                        v_mfma_f32_32x32x16, K split kRouterSplits ways into
//                        partial sums that the selection adds in fixed order
//                        (enough workgroups to stream the 2 MiB gate at 64
//                        tokens); each lane loads its operands directly, the
//                        next chunk's loads overlapping the current MFMAs.
//   router_select_kernel one wave per token: scores, top-k (DPP arg-max over
//                        (value, ~expert) keys), weights, slots.
#include "router_select.hpp"

namespace locali {

constexpr int kRouterSplits = 16;
constexpr int kRouterTokensPerPass = 8;
static_assert(kFusedSelectMaxTokens <= kRouterTokensPerPass, "fused selection needs the gemv path");

// --------------------------------------------------------------------------
// GEMV logits (decode).
// --------------------------------------------------------------------------
template <int GDT, bool XBF16>
__device__ __forceinline__ void gate_chunk(const void *w, int64_t off, uint32_t (&wp)[4], float (&wf)[8]) {
    if constexpr (GDT == 0) {
        const float4 a = *reinterpret_cast<const float4 *>(static_cast<const float *>(w) + off);
        const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(w) + off + 4);
        wf[0] = a.x; wf[1] = a.y; wf[2] = a.z; wf[3] = a.w;
        wf[4] = b.x; wf[5] = b.y; wf[6] = b.z; wf[7] = b.w;
    } else {
        const uint4 a = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(w) + off);
        wp[0] = a.x; wp[1] = a.y; wp[2] = a.z; wp[3] = a.w;
        if constexpr ((GDT == 2) != XBF16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                wf[2 * q] = GDT == 2 ? bf16_to_float(wp[q] & 0xffff) : f16_to_float(wp[q] & 0xffff);
                wf[2 * q + 1] = GDT == 2 ? bf16_to_float(wp[q] >> 16) : f16_to_float(wp[q] >> 16);
            }
        }
    }
}

constexpr int kRouterWaves = 4;   // experts per workgroup (one per wave)

// Fast path: gate and x share a 16-bit type (v_dot2), d = 512 * NCH, and TB
// tokens per pass. Every lane issues all NCH gate chunks of its expert and
// the TB tokens' x chunks before the first dot; tokens beyond L.tokens in
// the last pass re-read the last token and are not stored.
// One wave per workgroup: each expert's row then streams on its own compute
// unit (the 2 MiB gate spread over all of them; the workgroup -> XCD mapping
// is the same every step, so each gate row stays in one L2).
template <bool XBF16, int NCH, int TB>
__global__ __launch_bounds__(64) void router_gemv_fast_kernel(RouterLaunch L) {
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x;
    if (e >= L.E) return;
    u32x4 w[NCH];
    router_load_gate<NCH>(L, e, lane, w);
    for (int t0 = 0; t0 < L.tokens; t0 += TB) {
        float acc[TB];
        router_pass<XBF16, NCH, TB>(L, w, t0, lane, acc);
        const int q = lane / (64 / TB);
        if ((lane % (64 / TB)) == 0 && t0 + q < L.tokens)
            L.logits[static_cast<int64_t>(t0 + q) * L.E + e] = acc[0];
    }
}

// General path: any gate dtype (fp32, or a 16-bit type other than x's) and
// any d that is a multiple of 8.
template <int GDT, bool XBF16>
__global__ __launch_bounds__(64 * kRouterWaves) void router_gemv_kernel(RouterLaunch L) {
    constexpr int TB = kRouterTokensPerPass;
    constexpr bool kDot = GDT != 0 && ((GDT == 2) == XBF16);
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
    if (e < L.E) {
        for (int t0 = 0; t0 < L.tokens; t0 += TB) {
            float acc[TB];
#pragma unroll
            for (int q = 0; q < TB; ++q) acc[q] = 0.f;
            for (int k = lane * 8; k < L.d; k += 64 * 8) {
                uint32_t wp[4];
                float wf[8];
                gate_chunk<GDT, XBF16>(L.gate_w, static_cast<int64_t>(e) * L.d + k, wp, wf);
#pragma unroll
                for (int q = 0; q < TB; ++q) {
                    const uint4 xv = *reinterpret_cast<const uint4 *>(
                        L.x + static_cast<int64_t>(min(t0 + q, L.tokens - 1)) * L.d + k);
                    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
                    if constexpr (kDot) {
#pragma unroll
                        for (int u = 0; u < 4; ++u) acc[q] = dot2<XBF16>(xw[u], wp[u], acc[q]);
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            acc[q] = fmaf(to_float<XBF16>(static_cast<uint16_t>(xw[u])), wf[2 * u], acc[q]);
                            acc[q] = fmaf(to_float<XBF16>(static_cast<uint16_t>(xw[u] >> 16)),
                                          wf[2 * u + 1], acc[q]);
                        }
                    }
                }
            }
            reduce_transposed<TB, 64>(acc, lane);
            const int q = lane / (64 / TB);
            if ((lane % (64 / TB)) == 0 && t0 + q < L.tokens)
                L.logits[static_cast<int64_t>(t0 + q) * L.E + e] = acc[0];
        }
    }
}

// --------------------------------------------------------------------------
// MFMA logits for prefill: bf16/fp16 x and Wg of the same dtype.
// Workgroup: 4 waves; wave tile 32 tokens x 32 experts; workgroup tile
// 64 tokens x 64 experts; K split kRouterSplits ways over blockIdx.z.
// Partial logits land in L.logits[split][t][e].
// --------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <bool BF16>
__device__ __forceinline__ f32x16_t mfma32x32x16(u32x4 a, u32x4 b, f32x16_t c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                        __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                       __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

template <bool BF16>
__global__ __launch_bounds__(256) void router_mfma_kernel(RouterLaunch L) {
    // Each lane loads its own operands in the MFMA layout (A: token row
    // lane % 32, B: expert row lane % 32, 8 values at k + 8 (lane / 32)),
    // four MFMAs' worth a chunk, the next chunk's loads issued before the
    // current chunk's MFMAs; no LDS staging and no barrier, so a workgroup
    // waits for about one memory round trip. The loads are unconditional
    // (the last chunk's successor re-reads the last chunk).
    constexpr int CH = 4;                        // MFMAs per chunk
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
    const int split = blockIdx.z;
    const int kspan = L.d / kRouterSplits;
    const int nmf = kspan / 16;                  // MFMAs of the split, a multiple of CH
    const int wt = (wave & 1) * 32, we = (wave >> 1) * 32;   // wave sub-tile
    // rows past the tokens / experts repeat the last one; their results are
    // not stored
    const int tr = min(t0 + wt + (lane & 31), L.tokens - 1), er = min(e0 + we + (lane & 31), L.E - 1);
    const int koff = split * kspan + (lane >> 5) * 8;
    const uint16_t *xr = L.x + static_cast<int64_t>(tr) * L.d + koff;
    const uint16_t *wr = static_cast<const uint16_t *>(L.gate_w) + static_cast<int64_t>(er) * L.d + koff;
    u32x4 a0[CH], b0[CH], a1[CH], b1[CH];
    auto load = [&](u32x4(&a)[CH], u32x4(&b)[CH], int m0) {
        const int m = min(m0, nmf - CH);
#pragma unroll
        for (int q = 0; q < CH; ++q) {
            a[q] = *reinterpret_cast<const u32x4 *>(xr + 16 * (m + q));
            b[q] = *reinterpret_cast<const u32x4 *>(wr + 16 * (m + q));
        }
    };
    f32x16_t acc = {};
    auto run = [&](const u32x4(&a)[CH], const u32x4(&b)[CH]) {
#pragma unroll
        for (int q = 0; q < CH; ++q) acc = mfma32x32x16<BF16>(a[q], b[q], acc);
    };
    load(a0, b0, 0);
    for (int m = 0; m < nmf; m += 2 * CH) {
        load(a1, b1, m + CH);
        run(a0, b0);
        if (m + CH >= nmf) break;
        load(a0, b0, m + 2 * CH);
        run(a1, b1);
    }
    // D layout (32x32): lane holds column n = lane % 32 (expert) and rows
    // 8*(i/4) + 4*(lane/32) + (i%4) (tokens) for i < 16.
    float *out = L.logits + static_cast<int64_t>(split) * L.tokens * L.E;
    const int e = e0 + we + (lane & 31);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int t = t0 + wt + 8 * (i / 4) + 4 * (lane >> 5) + (i % 4);
        if (t < L.tokens && e < L.E) out[static_cast<int64_t>(t) * L.E + e] = acc[i];
    }
}

template <int NS, int SF, int M>
__global__ __launch_bounds__(256) void router_select_kernel(RouterLaunch L) {
    __shared__ float2 stage[4][64 * M];
    const int wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= L.tokens) return;
    const SelectOut o = select_token<NS, SF, M>(L, t, L.logits + static_cast<int64_t>(t) * L.E,
                                                static_cast<int64_t>(L.tokens) * L.E, stage[wave], L.top_k);
    select_store(L, t, o);
}

template <int NS, int SF>
hipError_t launch_select_m(const RouterLaunch &L, hipStream_t st) {
    const dim3 grid((L.tokens + 3) / 4), block(256);
    if (L.E <= 64) hipLaunchKernelGGL((router_select_kernel<NS, SF, 1>), grid, block, 0, st, L);
    else if (L.E <= 128) hipLaunchKernelGGL((router_select_kernel<NS, SF, 2>), grid, block, 0, st, L);
    else if (L.E <= 256) hipLaunchKernelGGL((router_select_kernel<NS, SF, 4>), grid, block, 0, st, L);
    else hipLaunchKernelGGL((router_select_kernel<NS, SF, 8>), grid, block, 0, st, L);
    return hipGetLastError();
}

template <int NS>
hipError_t launch_select(const RouterLaunch &L, hipStream_t st) {
    switch (L.score_func) {
    case 0: return launch_select_m<NS, 0>(L, st);
    case 1: return launch_select_m<NS, 1>(L, st);
    case 2: return launch_select_m<NS, 2>(L, st);
    default: return hipErrorInvalidValue;
    }
}

// --------------------------------------------------------------------------
hipError_t launch_router(const RouterLaunch &L, hipStream_t st, bool logits_only) {
    if (L.E > 64 * kRouterMaxExpertsPerLane || L.top_k > 16 || L.top_k < 1 || L.top_k > L.E)
        return hipErrorInvalidValue;
    const bool mfma_ok = !L.logits_in && L.tokens > kRouterTokensPerPass && L.gate_dtype != 0 &&
                         ((L.gate_dtype == 2) == L.x_bf16) && L.d % (64 * kRouterSplits) == 0;
    if (mfma_ok || L.logits_in) {
        if (L.logits_in) return launch_select<1>(L, st);
        dim3 grid((L.tokens + 63) / 64, (L.E + 63) / 64, kRouterSplits);
        if (L.x_bf16) hipLaunchKernelGGL(router_mfma_kernel<true>, grid, dim3(256), 0, st, L);
        else hipLaunchKernelGGL(router_mfma_kernel<false>, grid, dim3(256), 0, st, L);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_select<kRouterSplits>(L, st);
    }
    if (L.d % 8 != 0) return hipErrorInvalidValue;
    const int blocks = (L.E + kRouterWaves - 1) / kRouterWaves;
    dim3 grid(blocks), block(64 * kRouterWaves);
    const bool dot_ok = L.gate_dtype != 0 && ((L.gate_dtype == 2) == L.x_bf16);
    const int nch = L.d % 512 == 0 ? L.d / 512 : 0;
    if (dot_ok && (nch == 2 || nch == 4 || nch == 8 || nch == 16)) {
        const int tb = L.tokens == 1 ? 1 : L.tokens == 2 ? 2 : 4;
#define LOCALI_FAST(XB, N, T) \
    hipLaunchKernelGGL((router_gemv_fast_kernel<XB, N, T>), dim3(L.E), dim3(64), 0, st, L)
#define LOCALI_FAST_TB(XB, N) \
    if (tb == 1) LOCALI_FAST(XB, N, 1); else if (tb == 2) LOCALI_FAST(XB, N, 2); else LOCALI_FAST(XB, N, 4);
#define LOCALI_FAST_N(XB) \
    switch (nch) { case 2: LOCALI_FAST_TB(XB, 2) break; case 4: LOCALI_FAST_TB(XB, 4) break; \
                   case 8: LOCALI_FAST_TB(XB, 8) break; default: LOCALI_FAST_TB(XB, 16) break; }
        if (L.x_bf16) { LOCALI_FAST_N(true) } else { LOCALI_FAST_N(false) }
#undef LOCALI_FAST_N
#undef LOCALI_FAST_TB
#undef LOCALI_FAST
    } else {
#define LOCALI_ROUTER(GDT)                                                                  \
    if (L.x_bf16) hipLaunchKernelGGL((router_gemv_kernel<GDT, true>), grid, block, 0, st, L); \
    else hipLaunchKernelGGL((router_gemv_kernel<GDT, false>), grid, block, 0, st, L);
        switch (L.gate_dtype) {
        case 0: LOCALI_ROUTER(0); break;
        case 1: LOCALI_ROUTER(1); break;
        case 2: LOCALI_ROUTER(2); break;
        default: return hipErrorInvalidValue;
        }
#undef LOCALI_ROUTER
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || logits_only) return e;
    return launch_select<1>(L, st);
}

}  // namespace locali
