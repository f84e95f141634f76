// Decode-path expert kernels: one (token, expert) route per GEMV.
//
//   gateup_route_kernel   h[r, n] = swiglu(up_r(x_t)[n], gate_r(x_t)[n]) for
//                         every route r (routed top-k entries, then one
//                         shared-expert route per token). A workgroup of 8
//                         waves covers RB consecutive rows of one route: it
//                         prepares the token's activations into LDS while the
//                         slot's gate and up rows (J per wave) stream in, then
//                         consumes the rows in load order. The epilogue writes
//                         h and, because the workgroup owns whole words of the
//                         down projection's input, also h's prepared form.
//   down_combine_kernel   out[t, d] = round(sum_j round(round(y_j[d]) * w_j))
//                         (+ shared, rounded) for RB output rows d: one wave
//                         per route of token t streams the route's down rows
//                         against its prepared hidden vector; the route
//                         results meet in LDS and are combined in route
//                         order -- deterministic, no atomics.
// Reference arithmetic: dsv4_arena.py:168-235 (expert), arena.py:619-624 and
// dsv4_engine.py:259 (combine and shared expert).
#pragma once

#include "launch.hpp"
#include "qgemv.hpp"

namespace locali {

constexpr int kGateUpWaves = 8;

__device__ __forceinline__ void route_of(const RouteArgs &ra, int r, int &token, int &slot,
                                         bool &shared) {
    const int routed = ra.tokens * ra.top_k;
    shared = r >= routed;
    token = shared ? r - routed : r / ra.top_k;
    slot = shared ? 0 : ra.route_slot[r];
}

template <int LPR>
constexpr int gateup_rows_per_wave_load() { return LPR >= 16 ? 8 : LPR / 2; }

// ---------------------------------------------------------------------------
// SB: bits of the stored codes (BITS, or 3 for 3-bit rows widened to the
// 4-bit geometry on load).
template <int BITS, bool BF16, int CPL, int LPR, int GPC, int J, int SB = BITS>
__global__ __launch_bounds__(64 * kGateUpWaves) void gateup_route_kernel(
    RouteArgs ra, QProj gate, QProj up, QProj sgate, QProj sup, uint16_t *__restrict__ h,
    PrepVec hout, int down_bits, float limit, int fp32_swiglu) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    constexpr int RPW = J * G::kRPL;              // rows per wave
    constexpr int RB = kGateUpWaves * RPW;        // rows per workgroup
    constexpr int kUnits = LPR * CPL * 4;         // words of one row slice = prep units of x
    constexpr int kThreads = 64 * kGateUpWaves;
    constexpr int UPT = (kUnits + kThreads - 1) / kThreads;
    __shared__ __align__(16) uint16_t hs[RB];
    __shared__ XLds<BITS, BF16, CPL, LPR> xl;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lane_in_row = lane % LPR;
    const int row_sub = lane / LPR;
    const int r = blockIdx.y;
    int token, slot;
    bool shared;
    route_of(ra, r, token, slot, shared);
    // the route's projections field by field (a reference to one of two
    // parameter structs would make every field a dependent memory load);
    // the shared expert has the routed experts' shapes and quantisation
    const int N = gate.rows, K = gate.cols, group = gate.group;
    const int n0 = blockIdx.x * RB;
    const int row0 = n0 + wave * RPW;
    const bool active = row0 < N;
    const bool valid_slot = slot >= 0 && slot < (shared ? sgate.n_slots : gate.n_slots);
    const int sl = valid_slot ? slot : 0;
    const int64_t wpr = static_cast<int64_t>(K) * SB / 32;     // words per row
    const int gpr = K / group;                                  // groups per row

    // The token's activations first (loads retire in issue order, so rows
    // can be consumed as they land only if x is already in): each thread
    // reads the raw values of its prep unit(s) of the LDS prepared vector.
    constexpr int VPW = 32 / BITS;
    uint32_t xraw[UPT][VPW / 2];
    const uint16_t *xt = ra.x + static_cast<int64_t>(token) * K;
#pragma unroll
    for (int q = 0; q < UPT; ++q) {
        const int u = min(static_cast<int>(threadIdx.x) + q * kThreads, kUnits - 1);
        const int ul = u % LPR, uwd = (u / LPR) % 4, ui = u / (LPR * 4);
        const uint16_t *src = xt + (ul + LPR * ui) * G::kVPC + uwd * VPW;
#pragma unroll
        for (int c = 0; c < VPW / 8; ++c) {
            const uint4 a = reinterpret_cast<const uint4 *>(src)[c];
            xraw[q][4 * c] = a.x; xraw[q][4 * c + 1] = a.y; xraw[q][4 * c + 2] = a.z; xraw[q][4 * c + 3] = a.w;
        }
        if constexpr (VPW == 4) {
            const uint2 a = *reinterpret_cast<const uint2 *>(src);
            xraw[q][0] = a.x; xraw[q][1] = a.y;
        }
    }
    sched_fence();
    // Then every row's (small) metadata, then the weights in the order they
    // are consumed, so row j's math waits only for row j's chunk. The loads
    // are unconditional (rows clamped in range; a wave past the last row
    // re-reads it and stores nothing) so that the wait for x above does not
    // merge with a path on which no weight loads are outstanding.
    RowData<CPL, GPC> wg[J], wu[J];
    const int64_t w_slot = shared ? sgate.w_slot : gate.w_slot, m_slot = shared ? sgate.m_slot : gate.m_slot;
    const uint32_t *gw = (shared ? sgate.w : gate.w) + sl * w_slot, *uw = (shared ? sup.w : up.w) + sl * w_slot;
    const uint16_t *gs = (shared ? sgate.s : gate.s) + sl * m_slot, *gb = (shared ? sgate.b : gate.b) + sl * m_slot;
    const uint16_t *us = (shared ? sup.s : up.s) + sl * m_slot, *ub = (shared ? sup.b : up.b) + sl * m_slot;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int row = min(row0 + j * G::kRPL + row_sub, N - 1);
        load_row_meta<BITS, CPL, LPR, GPC>(wg[j], gs + row * gpr, gb + row * gpr, group,
                                           lane_in_row);
        load_row_meta<BITS, CPL, LPR, GPC>(wu[j], us + row * gpr, ub + row * gpr, group,
                                           lane_in_row);
    }
    sched_fence();
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int row = min(row0 + j * G::kRPL + row_sub, N - 1);
        load_row_weights<CPL, LPR, GPC, SB>(wg[j], gw + row * wpr, lane_in_row);
        load_row_weights<CPL, LPR, GPC, SB>(wu[j], uw + row * wpr, lane_in_row);
    }
    sched_fence();
    // Prepare x into LDS while the weights stream in (waits only for the x
    // loads issued above).
#pragma unroll
    for (int q = 0; q < UPT; ++q) {
        const int u = static_cast<int>(threadIdx.x) + q * kThreads;
        if (u < kUnits) {
            const int ul = u % LPR, uwd = (u / LPR) % 4, ui = u / (LPR * 4);
            prep_vals<BITS, BF16>(xraw[q], &xl.pairs[ui][uwd][0][ul], LPR, xl.part[ui][uwd][ul]);
        }
    }
    __syncthreads();
    if (active) {
        XVec<BITS, BF16, CPL, GPC> xv;
        load_xvec_lds<BITS, BF16, CPL, LPR, GPC>(xv, xl, lane_in_row);
        const uint32_t magic_v = opaque_vgpr(Pairs<BITS, BF16>::kMagic);
        float v[2 * J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            v[j] = row_partial<BITS, BF16, CPL, LPR, GPC>(wg[j], xv, magic_v);
            v[J + j] = row_partial<BITS, BF16, CPL, LPR, GPC>(wu[j], xv, magic_v);
        }
        reduce_transposed<2 * J, LPR>(v, lane);
        // lane holds value index vi = (lane % LPR) / (LPR / 2J): gates first.
        const float partner = shfl_xor(v[0], LPR / 2);
        constexpr int span = LPR / (2 * J);
        const int vi = lane_in_row / span;
        if (vi < J && (lane_in_row % span) == 0) {
            const int row = row0 + vi * G::kRPL + row_sub;
            if (row < N) {
                uint16_t out = 0;
                if (valid_slot)
                    out = swiglu16<BF16>(round16<BF16>(v[0]), round16<BF16>(partner), limit,
                                         fp32_swiglu != 0);
                h[static_cast<int64_t>(r) * N + row] = out;
                hs[row - n0] = out;
            }
        }
    }
    if (!hout.pairs) return;                      // uniform across the workgroup
    __syncthreads();
    // Prepared form of h for the down projection: this workgroup owns the
    // words covering rows [n0, n0 + RB).
    const int vpw = 32 / down_bits;
    const int nrows = min(RB, N - n0);
    const int words = nrows / vpw;
    if (static_cast<int>(threadIdx.x) < words) {
        const int unit = n0 / vpw + threadIdx.x;
        prep_unit_at<BF16>(down_bits, hs + threadIdx.x * vpw,
                           hout.pairs + r * hout.pairs_stride + unit * pairs_per_word<BF16>(down_bits),
                           hout.parts + r * hout.parts_stride + unit);
    }
}

// ---------------------------------------------------------------------------
template <int BITS, bool BF16, int CPL, int LPR, int GPC, int J, int WAVES, int SB = BITS>
__global__ __launch_bounds__(64 * WAVES) void down_combine_kernel(RouteArgs ra, QProj down,
                                                                   QProj sdown, PrepVec hin,
                                                                   CombineArgs ca) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    constexpr int RB = J * G::kRPL;               // rows per workgroup
    __shared__ float ylds[WAVES][RB];
    __shared__ float wlds[WAVES];   // the token's router weights, rounded to the activation dtype
    const int lane = threadIdx.x & 63;
    // wave index in an SGPR: the route's fields are then selected in scalar
    // registers (a reference to one of the two parameter structs would make
    // every field a dependent memory load)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane_in_row = lane % LPR;
    const int row_sub = lane / LPR;
    const int t = blockIdx.y;
    const int N = down.rows, K = down.cols;
    const int per_token = ra.top_k + ra.n_shared;
    const int routed = ra.tokens * ra.top_k;
    const int row0 = blockIdx.x * RB;
    const int64_t wpr = static_cast<int64_t>(K) * SB / 32;
    const int gpr = K / down.group;
    // the combine's weights are loaded first, so that the epilogue after the
    // barrier reads LDS instead of waiting on memory
    if (threadIdx.x < ra.top_k) wlds[threadIdx.x] = round16<BF16>(ca.weights[t * ra.top_k + threadIdx.x]);

    if (wave < per_token) {
        const int j = wave;
        const bool sh = j >= ra.top_k;
        const int r = sh ? routed + t : t * ra.top_k + j;
        // the route's prepared input first: it does not depend on the slot,
        // so its loads are in flight while the slot is looked up
        XVec<BITS, BF16, CPL, GPC> xv;
        load_xvec_global<BITS, BF16, CPL, LPR, GPC>(xv, hin.pairs + r * hin.pairs_stride,
                                                    hin.parts + r * hin.parts_stride, lane_in_row);
        sched_fence();
        const int slot = sh ? 0 : ra.route_slot[r];
        const bool valid_slot = slot >= 0 && slot < (sh ? sdown.n_slots : down.n_slots);
        const int sl = valid_slot ? slot : 0;
        const int group = sh ? sdown.group : down.group;
        const uint32_t *w = (sh ? sdown.w : down.w) + sl * (sh ? sdown.w_slot : down.w_slot);
        const int64_t m_slot = sh ? sdown.m_slot : down.m_slot;
        const uint16_t *s = (sh ? sdown.s : down.s) + sl * m_slot, *b = (sh ? sdown.b : down.b) + sl * m_slot;
        RowData<CPL, GPC> rd[J];
#pragma unroll
        for (int q = 0; q < J; ++q) {
            const int row = min(row0 + q * G::kRPL + row_sub, N - 1);
            load_row_meta<BITS, CPL, LPR, GPC>(rd[q], s + row * gpr, b + row * gpr, group, lane_in_row);
        }
        sched_fence();
#pragma unroll
        for (int q = 0; q < J; ++q) {
            const int row = min(row0 + q * G::kRPL + row_sub, N - 1);
            load_row_weights<CPL, LPR, GPC, SB>(rd[q], w + row * wpr, lane_in_row);
        }
        sched_fence();
        xvec_finish(xv);
        const uint32_t magic_v = opaque_vgpr(Pairs<BITS, BF16>::kMagic);
        float v[J];
#pragma unroll
        for (int q = 0; q < J; ++q) v[q] = row_partial<BITS, BF16, CPL, LPR, GPC>(rd[q], xv, magic_v);
        reduce_transposed<J, LPR>(v, lane);
        constexpr int span = LPR / J;
        const int vi = lane_in_row / span;
        if ((lane_in_row % span) == 0)
            ylds[j][vi * G::kRPL + row_sub] = valid_slot ? round16<BF16>(v[0]) : 0.f;
    }
    __syncthreads();
    // One thread advances the decode sync generation: the gate/up kernel of
    // this call has ended, and the next call's starts after this kernel. It
    // is issued after the workgroup's loads have landed, so that no load
    // waits behind it.
    if (ca.gen && (blockIdx.x | blockIdx.y | threadIdx.x) == 0)
        __hip_atomic_fetch_add(ca.gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int q = threadIdx.x; q < RB; q += blockDim.x) {
        const int row = row0 + q;
        if (row >= N) continue;
        float acc = 0.f;
        for (int j = 0; j < ra.top_k; ++j) {
            const float w = wlds[j];
            const float y = ylds[j][q];
            acc += ca.mode == 0 ? round16<BF16>(y * w) : y * w;
        }
        float out = round16<BF16>(acc);
        if (ra.n_shared) out = round16<BF16>(out + ylds[ra.top_k][q]);
        ca.out[static_cast<int64_t>(t) * N + row] = from_float<BF16>(out);
    }
}

// ---------------------------------------------------------------------------
// Templated launchers. Each (bits, dtype) pair is instantiated in its own
// translation unit (decode_b<bits>_<dtype>.hip) so the variants compile in
// parallel.
// ---------------------------------------------------------------------------
template <int BITS, bool BF16, int CPL, int LPR, int GPC, int SB = BITS>
hipError_t launch_gateup_t(const DecodeLaunch &L, hipStream_t st) {
    constexpr int J = gateup_rows_per_wave_load<LPR>();
    using G = Geom<BITS, CPL, LPR, GPC>;
    const int rows_per_block = kGateUpWaves * J * G::kRPL;
    // the epilogue prepares whole words of the down input, in the geometry the
    // down kernel computes in (4-bit for 3-bit codes)
    const int down_bits = lane_bits(L.down.bits);
    if (L.hprep.pairs && rows_per_block % (32 / down_bits)) return hipErrorInvalidValue;
    dim3 grid((L.gate.rows + rows_per_block - 1) / rows_per_block, L.routes);
    hipLaunchKernelGGL((gateup_route_kernel<BITS, BF16, CPL, LPR, GPC, J, SB>), grid,
                       dim3(64 * kGateUpWaves), 0, st, L.ra, L.gate, L.up, L.sgate, L.sup,
                       L.h, L.hprep, down_bits, L.limit, L.fp32_swiglu);
    return hipGetLastError();
}

template <int BITS, bool BF16, int CPL, int LPR, int GPC, int SB = BITS>
hipError_t launch_down_t(const DecodeLaunch &L, hipStream_t st) {
    constexpr int J = LPR >= 8 ? 8 : LPR;
    using G = Geom<BITS, CPL, LPR, GPC>;
    const int per_token = L.ra.top_k + L.ra.n_shared;
    const int rows_per_block = J * G::kRPL;
    dim3 grid((L.down.rows + rows_per_block - 1) / rows_per_block, L.ra.tokens);
    if (per_token <= 8) {
        hipLaunchKernelGGL((down_combine_kernel<BITS, BF16, CPL, LPR, GPC, J, 8, SB>), grid,
                           dim3(64 * per_token), 0, st, L.ra, L.down, L.sdown, L.hprep, L.ca);
    } else if (per_token <= 16) {
        hipLaunchKernelGGL((down_combine_kernel<BITS, BF16, CPL, LPR, GPC, J, 16, SB>), grid,
                           dim3(64 * per_token), 0, st, L.ra, L.down, L.sdown, L.hprep, L.ca);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// which: 0 = gate/up, 1 = down+combine. (CPL, LPR) from 16-byte chunks per row.
template <int BITS, bool BF16, int GPC, int SB = BITS>
hipError_t decode_geometry(int which, int cpr, const DecodeLaunch &L, hipStream_t st) {
#define LOCALI_GEOM(CPL, LPR)                                                  \
    return which == 0 ? launch_gateup_t<BITS, BF16, CPL, LPR, GPC, SB>(L, st)  \
                      : launch_down_t<BITS, BF16, CPL, LPR, GPC, SB>(L, st)
    switch (cpr) {
    case 8: LOCALI_GEOM(1, 8);
    case 16: LOCALI_GEOM(1, 16);
    case 32: LOCALI_GEOM(1, 32);
    case 64: LOCALI_GEOM(1, 64);
    case 128: LOCALI_GEOM(2, 64);
    case 256: LOCALI_GEOM(4, 64);
    default: return hipErrorInvalidValue;
    }
#undef LOCALI_GEOM
}

}  // namespace locali
