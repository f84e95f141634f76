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
//   router_gemv_kernel   one wave per expert (decode, few tokens): 16-byte
//                        loads of the gate row and of x, v_dot2 when x and Wg
//                        share a 16-bit type. The same launch prepares the
//                        activations for the expert kernels (prepared-vector
//                        form, see qgemv.hpp). The last wave to finish
//                        (device-scope counter) selects for every token, so
//                        decode routing is a single launch.
//   router_mfma_kernel   prefill: 32 tokens x 32 experts per wave with
//                        v_mfma_f32_32x32x16, K split kRouterSplits ways into
//                        partial sums that the selection adds in fixed order.
//   router_select_kernel one wave per token: scores, top-k, weights, slots.
//   prep_vectors_kernel  standalone activation prep for the expert kernels.
#include "launch.hpp"

namespace locali {

constexpr int kRouterMaxExpertsPerLane = 8;   // E <= 512
constexpr int kRouterSplits = 4;
constexpr int kRouterTokensPerPass = 8;

__device__ __forceinline__ float softplus_f(float l) {
    return l > 20.0f ? l : log1pf(expf(l));
}

// --------------------------------------------------------------------------
// Selection for one token, executed by one full wave. Lane j < top_k ends up
// owning the j-th choice.
// --------------------------------------------------------------------------
__device__ void select_token(const RouterLaunch &L, int t, const float *logit_row, int nsplit,
                             int64_t split_stride) {
    const int lane = threadIdx.x & 63;
    float sc[kRouterMaxExpertsPerLane], sel[kRouterMaxExpertsPerLane];
    float lmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < kRouterMaxExpertsPerLane; ++i) {
        const int e = lane + 64 * i;
        float l = -INFINITY;
        if (e < L.E) {
            if (L.logits_in) {
                l = L.logits_in[static_cast<int64_t>(t) * L.E + e];
            } else {
                l = 0.f;
                for (int s = 0; s < nsplit; ++s) l += logit_row[s * split_stride + e];
            }
        }
        sc[i] = l;
        lmax = fmaxf(lmax, l);
    }
    float denom = 1.f;
    if (L.score_func == 2) {
        for (int m = 32; m >= 1; m >>= 1) lmax = fmaxf(lmax, __shfl_xor(lmax, m, 64));
        float z = 0.f;
#pragma unroll
        for (int i = 0; i < kRouterMaxExpertsPerLane; ++i)
            if (lane + 64 * i < L.E) z += expf(sc[i] - lmax);
        for (int m = 32; m >= 1; m >>= 1) z += __shfl_xor(z, m, 64);
        denom = z;
    }
#pragma unroll
    for (int i = 0; i < kRouterMaxExpertsPerLane; ++i) {
        const int e = lane + 64 * i;
        if (e < L.E) {
            const float l = sc[i];
            float s;
            if (L.score_func == 0) s = sqrtf(softplus_f(l));
            else if (L.score_func == 1) s = 1.0f / (1.0f + expf(-l));
            else s = expf(l - lmax) / denom;
            sc[i] = s;
            sel[i] = s + (L.bias ? L.bias[e] : 0.f);
        } else {
            sc[i] = 0.f;
            sel[i] = -INFINITY;
        }
    }
    int my_e = -1;
    float my_s = 0.f;
    for (int j = 0; j < L.top_k; ++j) {
        int best_e;
        if (L.tid2eid) {
            const int id = L.input_ids[t];
            best_e = (id >= 0 && id < L.vocab) ? L.tid2eid[static_cast<int64_t>(id) * L.top_k + j] : -1;
            if (best_e >= L.E) best_e = -1;
        } else {
            float bv = -INFINITY;
            int be = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < kRouterMaxExpertsPerLane; ++i) {
                const int e = lane + 64 * i;
                if (e < L.E && (sel[i] > bv || (sel[i] == bv && e < be))) { bv = sel[i]; be = e; }
            }
            for (int m = 32; m >= 1; m >>= 1) {
                const float ov = __shfl_xor(bv, m, 64);
                const int oe = __shfl_xor(be, m, 64);
                if (ov > bv || (ov == bv && oe < be)) { bv = ov; be = oe; }
            }
            best_e = be < L.E ? be : -1;
#pragma unroll
            for (int i = 0; i < kRouterMaxExpertsPerLane; ++i)
                if (lane + 64 * i == best_e) sel[i] = -INFINITY;
        }
        float mine = 0.f;
        const int slot_i = best_e >= 0 ? (best_e >> 6) : 0;
#pragma unroll
        for (int i = 0; i < kRouterMaxExpertsPerLane; ++i)
            if (i == slot_i) mine = sc[i];
        const float s = best_e >= 0 ? __shfl(mine, best_e & 63, 64) : 0.f;
        if (lane == j) {
            my_e = best_e;
            my_s = s;
        }
    }
    float sum = lane < L.top_k ? my_s : 0.f;
    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 64);
    if (lane < L.top_k) {
        float w = my_s;
        if (L.norm_topk) w = w / (sum + 1e-20f);
        const int64_t o = static_cast<int64_t>(t) * L.top_k + lane;
        L.idx[o] = my_e;
        L.weights[o] = w * L.routed_scale;
        if (L.route_slot) {
            int slot = -1;
            if (my_e >= 0 && L.slot_of_expert) slot = L.slot_of_expert[my_e];
            if (slot >= L.n_slots) slot = -1;
            L.route_slot[o] = slot;
        }
    }
}

// --------------------------------------------------------------------------
// Activation prep (prepared-vector form of qgemv.hpp) for n_vec rows of v.
// --------------------------------------------------------------------------
template <bool BF16>
__device__ __forceinline__ void prep_units(const uint16_t *v, int n_vec, int K, int bits,
                                           const PrepVec &out, int first, int count) {
    const int vpw = 32 / bits;
    const int per_vec = K / vpw;
    const int ppw = pairs_per_word<BF16>(bits);
    for (int u = first; u < first + count && u < n_vec * per_vec; u += 1) {
        const int vec = u / per_vec, unit = u % per_vec;
        prep_unit_at<BF16>(bits, v + static_cast<int64_t>(vec) * K + unit * vpw,
                           out.pairs + vec * out.pairs_stride + unit * ppw,
                           out.parts + vec * out.parts_stride + unit);
    }
}

template <bool BF16>
__global__ __launch_bounds__(256) void prep_vectors_kernel(const uint16_t *v, int n_vec, int K,
                                                           int bits, PrepVec out) {
    const int u = blockIdx.x * blockDim.x + threadIdx.x;
    prep_units<BF16>(v, n_vec, K, bits, out, u, 1);
}

hipError_t launch_prep_vectors(const uint16_t *v, int n_vec, int K, int bits, bool bf16, PrepVec out,
                               hipStream_t st) {
    const int units = n_vec * (K * bits / 32);
    dim3 grid((units + 255) / 256);
    if (bf16) hipLaunchKernelGGL(prep_vectors_kernel<true>, grid, dim3(256), 0, st, v, n_vec, K, bits, out);
    else hipLaunchKernelGGL(prep_vectors_kernel<false>, grid, dim3(256), 0, st, v, n_vec, K, bits, out);
    return hipGetLastError();
}

// --------------------------------------------------------------------------
// GEMV logits (decode) + activation prep + fused last-wave selection.
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

constexpr int kRouterWaves = 8;   // experts per workgroup (one per wave)

template <int GDT, bool XBF16>
__global__ __launch_bounds__(64 * kRouterWaves) void router_gemv_kernel(RouterLaunch L) {
    constexpr int TB = kRouterTokensPerPass;
    constexpr bool kDot = GDT != 0 && ((GDT == 2) == XBF16);
    const int lane = threadIdx.x & 63;
    const int e = blockIdx.x * kRouterWaves + (threadIdx.x >> 6);
    if (L.xprep.pairs)
        prep_units<XBF16>(L.x, L.tokens, L.d, L.prep_bits, L.xprep,
                          blockIdx.x * blockDim.x + threadIdx.x, 1);
    if (!L.logits_in && e < L.E) {
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
                    if (t0 + q < L.tokens) {
                        const uint4 xv = *reinterpret_cast<const uint4 *>(
                            L.x + static_cast<int64_t>(t0 + q) * L.d + k);
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
            }
            reduce_transposed<TB, 64>(acc, lane);
            const int q = lane / (64 / TB);
            if ((lane % (64 / TB)) == 0 && t0 + q < L.tokens)
                L.logits[static_cast<int64_t>(t0 + q) * L.E + e] = acc[0];
        }
    }
    // Last workgroup to arrive selects: release this workgroup's logits,
    // count once per workgroup (device-scope atomics are costly, so only
    // E / 8 of them), and let the final arrival acquire everyone's.
    __shared__ unsigned last;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(L.counter, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int t = threadIdx.x >> 6; t < L.tokens; t += kRouterWaves)
        select_token(L, t, L.logits + static_cast<int64_t>(t) * L.E, 1, 0);
    if (threadIdx.x == 0) atomicExch(L.counter, 0u);
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
    constexpr int KT = 64;                       // K per LDS stage
    constexpr int PAD = 8;                       // 16-bit elements of row padding
    __shared__ uint16_t xs[64][KT + PAD];
    __shared__ uint16_t ws[64][KT + PAD];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
    const int split = blockIdx.z;
    const int kspan = L.d / kRouterSplits;
    const int kbeg = split * kspan, kend = kbeg + kspan;
    const uint16_t *gw = static_cast<const uint16_t *>(L.gate_w);
    const int wt = (wave & 1) * 32, we = (wave >> 1) * 32;   // wave sub-tile
    f32x16_t acc = {};
    for (int k0 = kbeg; k0 < kend; k0 += KT) {
        for (int c = threadIdx.x; c < 64 * KT / 8; c += 256) {
            const int row = c / (KT / 8), col = (c % (KT / 8)) * 8;
            uint4 xv = make_uint4(0, 0, 0, 0), wv = make_uint4(0, 0, 0, 0);
            if (t0 + row < L.tokens)
                xv = *reinterpret_cast<const uint4 *>(L.x + static_cast<int64_t>(t0 + row) * L.d + k0 + col);
            if (e0 + row < L.E)
                wv = *reinterpret_cast<const uint4 *>(gw + static_cast<int64_t>(e0 + row) * L.d + k0 + col);
            *reinterpret_cast<uint4 *>(&xs[row][col]) = xv;
            *reinterpret_cast<uint4 *>(&ws[row][col]) = wv;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < KT; kk += 16) {
            const int kofs = kk + (lane >> 5) * 8;
            const u32x4 a = *reinterpret_cast<const u32x4 *>(&xs[wt + (lane & 31)][kofs]);
            const u32x4 b = *reinterpret_cast<const u32x4 *>(&ws[we + (lane & 31)][kofs]);
            acc = mfma32x32x16<BF16>(a, b, acc);
        }
        __syncthreads();
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

__global__ __launch_bounds__(256) void router_select_kernel(RouterLaunch L, int nsplit) {
    const int wave = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wave;
    if (t >= L.tokens) return;
    select_token(L, t, L.logits + static_cast<int64_t>(t) * L.E, nsplit,
                 static_cast<int64_t>(L.tokens) * L.E);
}

// --------------------------------------------------------------------------
hipError_t launch_router(const RouterLaunch &L, hipStream_t st) {
    if (L.E > 64 * kRouterMaxExpertsPerLane || L.top_k > 16 || L.top_k < 1 || L.top_k > L.E)
        return hipErrorInvalidValue;
    const bool mfma_ok = !L.logits_in && L.tokens > kRouterTokensPerPass && L.gate_dtype != 0 &&
                         ((L.gate_dtype == 2) == L.x_bf16) && L.d % (64 * kRouterSplits) == 0;
    if (mfma_ok) {
        if (L.xprep.pairs) {
            hipError_t e = launch_prep_vectors(L.x, L.tokens, L.d, L.prep_bits, L.x_bf16, L.xprep, st);
            if (e != hipSuccess) return e;
        }
        dim3 grid((L.tokens + 63) / 64, (L.E + 63) / 64, kRouterSplits);
        if (L.x_bf16) hipLaunchKernelGGL(router_mfma_kernel<true>, grid, dim3(256), 0, st, L);
        else hipLaunchKernelGGL(router_mfma_kernel<false>, grid, dim3(256), 0, st, L);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(router_select_kernel, dim3((L.tokens + 3) / 4), dim3(256), 0, st, L,
                           kRouterSplits);
        return hipGetLastError();
    }
    if (L.d % 8 != 0) return hipErrorInvalidValue;
    // every wave must cover its share of the prep units
    const int blocks = (L.E + kRouterWaves - 1) / kRouterWaves;
    if (L.xprep.pairs && static_cast<int64_t>(blocks) * 64 * kRouterWaves <
                             static_cast<int64_t>(L.tokens) * (L.d * L.prep_bits / 32)) {
        hipError_t e = launch_prep_vectors(L.x, L.tokens, L.d, L.prep_bits, L.x_bf16, L.xprep, st);
        if (e != hipSuccess) return e;
        RouterLaunch L2 = L;
        L2.xprep.pairs = nullptr;
        return launch_router(L2, st);
    }
    dim3 grid(blocks), block(64 * kRouterWaves);
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
    return hipGetLastError();
}

}  // namespace locali
