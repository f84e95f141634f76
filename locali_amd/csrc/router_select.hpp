// Top-k selection of one token by one wave: scores, selection-only bias,
// top-k, renormalisation and routed scaling, slot lookup. Shared by the router
// select kernel and the decode gate/up kernel that selects for its own token.
// Semantics follow the DeepSeek-V4 gate the reference module delegates to
// (dsv4_arena.py:147-153, 165-166) and Locali's sigmoid router
// (arena.py:501-506); in-row order is canonical (descending selection value,
// ties to the lower expert id).
#pragma once

#include "launch.hpp"

namespace locali {

constexpr int kRouterMaxExpertsPerLane = 8;   // E <= 512

// --------------------------------------------------------------------------
// Selection for one token, executed by one full wave. Lane j < top_k ends up
// owning the j-th choice. Logits are the sum of NS partial rows (fixed order)
// at logit_row + s * split_stride, or L.logits_in when given. Lane l holds
// experts l + 64 i, i < M (M = ceil(E / 64)); SF is the score function.
// A lone wave pays for every instruction and every memory round trip, so:
// everything the selection can need (logits, bias, the expert -> slot map,
// the hash row) is loaded up front at clamped in-bounds addresses; scores use
// the hardware exp/log; each lane sorts its M keys once, after which a round
// of top-k is one wave-wide arg-max of the lane heads (two 32-bit maxima
// that stay in the vector unit) plus a pop; scores and
// slots of the chosen experts are fetched back from LDS (`stage`, 64 * M
// float2 per wave) by the owning lanes.
// --------------------------------------------------------------------------
template <int SF>
__device__ __forceinline__ float score_of(float l, float lmax, float denom) {
    if constexpr (SF == 0) {
        // sqrt(softplus(l)); log1p(e) ~ e within 1.5e-7 relative below -15
        const float e = __expf(l);
        const float sp = l > 20.0f ? l : (l < -15.0f ? e : __logf(1.0f + e));
        return __builtin_amdgcn_sqrtf(sp);   // hardware square root (1 ulp)
    } else if constexpr (SF == 1) {
        return 1.0f / (1.0f + __expf(-l));
    } else {
        return __expf(l - lmax) / denom;
    }
}

__device__ __forceinline__ bool key_gt(uint32_t ah, uint32_t al, uint32_t bh, uint32_t bl) {
    return ah > bh || (ah == bh && al > bl);
}

// The choice owned by lane j < top_k: expert (-1: none), its slot (-1: no
// slot) and its weight.
struct SelectOut {
    int e, slot;
    float w;
};

// What the selection needs besides the logits, loaded up front at clamped
// in-bounds addresses: selection bias, the expert -> slot map and the hash row.
template <int M>
struct SelectInputs {
    float bias[M];
    int slot_of[M];
    int hash_e;
};

template <int M>
__device__ __forceinline__ void select_inputs(const RouterLaunch &L, int t, SelectInputs<M> &in) {
    const int lane = threadIdx.x & 63;
    in.hash_e = -1;
    if (L.tid2eid) {
        const int id = L.input_ids[t];
        if (id >= 0 && id < L.vocab && lane < L.top_k)
            in.hash_e = L.tid2eid[static_cast<int64_t>(id) * L.top_k + lane];
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int e = min(lane + 64 * i, L.E - 1);
        in.bias[i] = L.bias ? L.bias[e] : 0.f;
        in.slot_of[i] = L.slot_of_expert ? L.slot_of_expert[e] : -1;
    }
}

// The selection proper on the token's logits (lane l holds experts l + 64 i).
template <int SF, int M>
__device__ SelectOut select_core(const RouterLaunch &L, const float (&lg)[M], const SelectInputs<M> &in,
                                 float2 *stage, int rounds) {
    const int lane = threadIdx.x & 63;
    float sc[M];
#pragma unroll
    for (int i = 0; i < M; ++i) sc[i] = lane + 64 * i < L.E ? lg[i] : -INFINITY;
    float denom = 1.f, lmax = -INFINITY;
    if constexpr (SF == 2) {
#pragma unroll
        for (int i = 0; i < M; ++i) lmax = fmaxf(lmax, sc[i]);
        for (int m = 32; m >= 1; m >>= 1) lmax = fmaxf(lmax, __shfl_xor(lmax, m, 64));
        float z = 0.f;
#pragma unroll
        for (int i = 0; i < M; ++i) z += lane + 64 * i < L.E ? __expf(sc[i] - lmax) : 0.f;
        for (int m = 32; m >= 1; m >>= 1) z += __shfl_xor(z, m, 64);
        denom = z;
    }
    // Keys: hi = ordered selection value, lo = ~expert (ties -> lower id);
    // (0, 0) marks an invalid candidate.
    uint32_t kh[M], kl[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int e = lane + 64 * i;
        const bool valid = e < L.E;
        const float s = score_of<SF>(valid ? sc[i] : 0.f, lmax, denom);
        stage[e] = make_float2(s, __int_as_float(in.slot_of[i]));
        kh[i] = valid ? ordered_bits(s + in.bias[i]) : 0u;
        kl[i] = valid ? ~static_cast<uint32_t>(e) : 0u;
    }
    // Sort the lane's keys descending (insertion network, M <= 8).
#pragma unroll
    for (int i = 1; i < M; ++i) {
#pragma unroll
        for (int j = i; j > 0; --j) {
            const bool sw = key_gt(kh[j], kl[j], kh[j - 1], kl[j - 1]);
            const uint32_t th = kh[j], tl = kl[j];
            kh[j] = sw ? kh[j - 1] : th;
            kl[j] = sw ? kl[j - 1] : tl;
            kh[j - 1] = sw ? th : kh[j - 1];
            kl[j - 1] = sw ? tl : kl[j - 1];
        }
    }
    // rounds < top_k: only the first `rounds` choices (and their slots) are
    // needed; later lanes keep expert -1 and the weights are not final
    int my_e = -1;
    for (int j = 0; j < rounds; ++j) {
        int best_e;
        if (L.tid2eid) {
            best_e = __builtin_amdgcn_readlane(in.hash_e, j);
            if (best_e >= L.E || best_e < 0) best_e = -1;
        } else {
            uint32_t bh = kh[0], bl = kl[0];
            wave_max_key(bh, bl);
            best_e = bh == 0 && bl == 0 ? -1 : static_cast<int>(~bl);
            // the winner pops its head (keys are unique: lo holds the expert)
            const bool pop = kh[0] == bh && kl[0] == bl && best_e >= 0;
#pragma unroll
            for (int i = 0; i + 1 < M; ++i) {
                kh[i] = pop ? kh[i + 1] : kh[i];
                kl[i] = pop ? kl[i + 1] : kl[i];
            }
            kh[M - 1] = pop ? 0u : kh[M - 1];
            kl[M - 1] = pop ? 0u : kl[M - 1];
        }
        if (lane == j) my_e = best_e;
    }
    __builtin_amdgcn_wave_barrier();
    float my_s = 0.f;
    int my_slot = -1;
    if (lane < L.top_k && my_e >= 0) {
        const float2 v = stage[my_e];
        my_s = v.x;
        my_slot = __float_as_int(v.y);
    }
    float sum = 0.f;   // selection order, as the scores are gathered
    for (int j = 0; j < L.top_k; ++j)
        sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_s), j));
    SelectOut o;
    o.e = my_e;
    o.slot = my_e < 0 || my_slot >= L.n_slots ? -1 : my_slot;
    float w = my_s;
    if (L.norm_topk) w = w / (sum + 1e-20f);
    o.w = w * L.routed_scale;
    return o;
}

template <int NS, int SF, int M>
__device__ SelectOut select_token(const RouterLaunch &L, int t, const float *logit_row, int64_t split_stride,
                                  float2 *stage, int rounds) {
    const int lane = threadIdx.x & 63;
    float part[NS][M];
    SelectInputs<M> in;
    select_inputs<M>(L, t, in);
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int e = min(lane + 64 * i, L.E - 1);
        if (L.logits_in) {
            part[0][i] = L.logits_in[static_cast<int64_t>(t) * L.E + e];
#pragma unroll
            for (int q = 1; q < NS; ++q) part[q][i] = 0.f;
        } else {
#pragma unroll
            for (int q = 0; q < NS; ++q) part[q][i] = logit_row[q * split_stride + e];
        }
    }
    float lg[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        float l = part[0][i];
#pragma unroll
        for (int q = 1; q < NS; ++q) l += part[q][i];
        lg[i] = l;
    }
    return select_core<SF, M>(L, lg, in, stage, rounds);
}

// ---------------------------------------------------------------------------
// Logits handed from the router rows of the fused decode kernel: word e of a
// token's row is (tag << 32) | fp32 bits, written by one relaxed agent-scope
// 64-bit store, so a word is either wholly this call's or stale. The wave
// polls the row (relaxed agent-scope loads: coherent across the XCDs' L2s)
// until every word carries `tag`, sleeping between polls. Bounded: after
// kSyncMaxSpins polls it gives up and returns false.
constexpr uint32_t kSyncMaxSpins = 1u << 18;

template <int M>
__device__ __forceinline__ bool poll_logits(const uint64_t *row, int E, uint32_t tag, float (&lg)[M]) {
    const int lane = threadIdx.x & 63;
    // while the logits are still being computed, poll one word (the row's
    // last expert; every lane reads the same address: one request a wave)
    // instead of the whole row, so that hundreds of polling waves do not
    // load the memory path the router rows' stores and weights take
    for (uint32_t spin = 0; spin < kSyncMaxSpins; ++spin) {
        const uint64_t w = __hip_atomic_load(row + (E - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (static_cast<uint32_t>(w >> 32) == tag) break;
        __builtin_amdgcn_s_sleep(1);
    }
    for (uint32_t spin = 0;; ++spin) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < M; ++i) {
            const uint64_t v = __hip_atomic_load(row + min(lane + 64 * i, E - 1), __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            ok = ok && static_cast<uint32_t>(v >> 32) == tag;
            lg[i] = __uint_as_float(static_cast<uint32_t>(v));
        }
        if (__all(ok)) return true;
        if (spin >= kSyncMaxSpins) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

// select_token on logits polled from the sync row of token t. If they never
// arrive the token gets no routes (expert -1, slot -1, weight 0).
template <int SF, int M>
__device__ SelectOut select_token_polled(const RouterLaunch &L, int t, uint32_t tag, float2 *stage, int rounds) {
    SelectInputs<M> in;
    select_inputs<M>(L, t, in);
    float lg[M];
    if (!poll_logits<M>(L.sync_logits + static_cast<int64_t>(t) * L.E, L.E, tag, lg)) {
        SelectOut o;
        o.e = -1;
        o.slot = -1;
        o.w = 0.f;
        return o;
    }
    return select_core<SF, M>(L, lg, in, stage, rounds);
}

template <int M>
__device__ SelectOut select_token_polled_any(const RouterLaunch &L, int t, uint32_t tag, float2 *stage, int rounds) {
    switch (L.score_func) {
    case 0: return select_token_polled<0, M>(L, t, tag, stage, rounds);
    case 1: return select_token_polled<1, M>(L, t, tag, stage, rounds);
    default: return select_token_polled<2, M>(L, t, tag, stage, rounds);
    }
}

// ---------------------------------------------------------------------------
// Router logits of one expert by one wave: the lane's NCH 16-byte chunks of
// the gate row (router_load_gate), then per pass of TB tokens (tokens past
// L.tokens re-read the last one) the x chunks, the dots and a transposed
// reduction after which lane q * (64 / TB) holds token t0 + q's logit. The
// logits kernel and the fused decode kernel both use these, so their logits
// are the same bits.
template <int NCH>
__device__ __forceinline__ void router_load_gate(const RouterLaunch &L, int e, int lane, u32x4 (&w)[NCH]) {
    const uint16_t *gw = static_cast<const uint16_t *>(L.gate_w) + static_cast<int64_t>(e) * L.d;
#pragma unroll
    for (int i = 0; i < NCH; ++i)
        // ordinary (cacheable) loads: the gate is read again on every token,
        // while the expert weights streamed between its uses are non-temporal
        w[i] = reinterpret_cast<const u32x4 *>(gw)[lane + 64 * i];
}

template <bool XBF16, int NCH, int TB>
__device__ __forceinline__ void router_pass(const RouterLaunch &L, const u32x4 (&w)[NCH], int t0, int lane,
                                            float (&acc)[TB]) {
    uint4 xv[TB][NCH];
#pragma unroll
    for (int q = 0; q < TB; ++q) {
        const uint16_t *xr = L.x + static_cast<int64_t>(min(t0 + q, L.tokens - 1)) * L.d;
#pragma unroll
        for (int i = 0; i < NCH; ++i) xv[q][i] = reinterpret_cast<const uint4 *>(xr)[lane + 64 * i];
    }
#pragma unroll
    for (int q = 0; q < TB; ++q) {
        acc[q] = 0.f;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            acc[q] = dot2<XBF16>(xv[q][i].x, w[i].x, acc[q]);
            acc[q] = dot2<XBF16>(xv[q][i].y, w[i].y, acc[q]);
            acc[q] = dot2<XBF16>(xv[q][i].z, w[i].z, acc[q]);
            acc[q] = dot2<XBF16>(xv[q][i].w, w[i].w, acc[q]);
        }
    }
    reduce_transposed<TB, 64>(acc, lane);
}

// Stores token t's choices (lanes < top_k).
__device__ __forceinline__ void select_store(const RouterLaunch &L, int t, const SelectOut &o) {
    const int lane = threadIdx.x & 63;
    if (lane < L.top_k) {
        const int64_t i = static_cast<int64_t>(t) * L.top_k + lane;
        L.idx[i] = o.e;
        L.weights[i] = o.w;
        if (L.route_slot) L.route_slot[i] = o.slot;
    }
}

// Score function chosen at run time (for kernels that select on the side).
template <int NS, int M>
__device__ SelectOut select_token_any(const RouterLaunch &L, int t, const float *logit_row,
                                      int64_t split_stride, float2 *stage, int rounds) {
    switch (L.score_func) {
    case 0: return select_token<NS, 0, M>(L, t, logit_row, split_stride, stage, rounds);
    case 1: return select_token<NS, 1, M>(L, t, logit_row, split_stride, stage, rounds);
    default: return select_token<NS, 2, M>(L, t, logit_row, split_stride, stage, rounds);
    }
}


}  // namespace locali
