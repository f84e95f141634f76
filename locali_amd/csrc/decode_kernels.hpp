// Decode-path expert kernels: one (token, expert) route per GEMV.
//
//   gateup_route_kernel   h[r, n] = swiglu(up_r(x_t)[n], gate_r(x_t)[n])
//                         for every route r (routed top-k entries, then one
//                         shared-expert route per token), streaming the gate
//                         and up rows of the route's arena slot.
//   down_combine_kernel   out[t, d] = sum_j round(round(down_j(h_j)[d]) * w_j)
//                         (+ shared) for a block of output rows d; all routes
//                         of token t run in the same workgroup (one wave per
//                         route) and are combined through LDS in route order,
//                         so the result is deterministic without atomics.
// Reference arithmetic: dsv4_arena.py:168-235 (expert), arena.py:619-624 and
// dsv4_engine.py:259 (combine and shared expert).
#pragma once

#include "launch.hpp"
#include "qgemv.hpp"

namespace locali {

__device__ __forceinline__ void route_of(const RouteArgs &ra, int r, int &token, int &slot,
                                         bool &shared) {
    const int routed = ra.tokens * ra.top_k;
    shared = r >= routed;
    token = shared ? r - routed : r / ra.top_k;
    slot = shared ? 0 : ra.route_slot[r];
}

// ---------------------------------------------------------------------------
template <int BITS, bool BF16, int CPL, int LPR, int GPC, int J>
__global__ __launch_bounds__(256) void gateup_route_kernel(RouteArgs ra, QProj gate, QProj up,
                                                            QProj sgate, QProj sup,
                                                            uint16_t *__restrict__ h,
                                                            float limit, int fp32_swiglu) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    constexpr int RPW = J * G::kRPL;           // rows per wave
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lane_in_row = lane % LPR;
    const int row_sub = lane / LPR;
    const int r = blockIdx.y;
    int token, slot;
    bool shared;
    route_of(ra, r, token, slot, shared);
    const QProj &pg = shared ? sgate : gate;
    const QProj &pu = shared ? sup : up;
    const int N = pg.rows, K = pg.cols;
    const int row0 = (blockIdx.x * (blockDim.x >> 6) + wave) * RPW;
    if (row0 >= N) return;
    const bool valid_slot = slot >= 0 && slot < pg.n_slots;

    XVec<BITS, BF16, CPL, GPC> xv;
    load_xvec<BITS, BF16, CPL, LPR, GPC>(xv, ra.x + static_cast<int64_t>(token) * K, lane_in_row);

    const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;   // words per row
    const int gpr = K / pg.group;                               // groups per row
    const int sl = valid_slot ? slot : 0;
    const uint32_t *gw = pg.w + sl * pg.w_slot;
    const uint32_t *uw = pu.w + sl * pu.w_slot;
    const uint16_t *gs = pg.s + sl * pg.m_slot, *gb = pg.b + sl * pg.m_slot;
    const uint16_t *us = pu.s + sl * pu.m_slot, *ub = pu.b + sl * pu.m_slot;

    RowChunks<CPL> wg[J], wu[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int row = min(row0 + j * G::kRPL + row_sub, N - 1);
        load_row<BITS, CPL, LPR>(wg[j], gw + row * wpr, lane_in_row);
        load_row<BITS, CPL, LPR>(wu[j], uw + row * wpr, lane_in_row);
    }
    float v[2 * J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int row = min(row0 + j * G::kRPL + row_sub, N - 1);
        v[j] = row_partial<BITS, BF16, CPL, LPR, GPC>(wg[j], xv, gs + row * gpr, gb + row * gpr,
                                                       pg.group, lane_in_row);
        v[J + j] = row_partial<BITS, BF16, CPL, LPR, GPC>(wu[j], xv, us + row * gpr,
                                                           ub + row * gpr, pu.group, lane_in_row);
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
        }
    }
}

// ---------------------------------------------------------------------------
constexpr int kMaxRoutesPerToken = 16;

template <int BITS, bool BF16, int CPL, int LPR, int GPC, int J>
__global__ __launch_bounds__(1024) void down_combine_kernel(RouteArgs ra, QProj down, QProj sdown,
                                                             const uint16_t *__restrict__ h,
                                                             CombineArgs ca) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    constexpr int RPW = J * G::kRPL;           // rows per workgroup (all waves share them)
    __shared__ float ylds[kMaxRoutesPerToken][RPW];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nwaves = blockDim.x >> 6;
    const int lane_in_row = lane % LPR;
    const int row_sub = lane / LPR;
    const int t = blockIdx.y;
    const int N = down.rows, K = down.cols;
    const int row0 = blockIdx.x * RPW;
    const int per_token = ra.top_k + ra.n_shared;
    const int routed = ra.tokens * ra.top_k;
    const int64_t wpr = static_cast<int64_t>(K) * BITS / 32;
    const int gpr = K / down.group;

    for (int j = wave; j < per_token; j += nwaves) {
        const bool shared = j >= ra.top_k;
        const int r = shared ? routed + t : t * ra.top_k + j;
        const int slot = shared ? 0 : ra.route_slot[r];
        const QProj &p = shared ? sdown : down;
        const bool valid_slot = slot >= 0 && slot < p.n_slots;
        const int sl = valid_slot ? slot : 0;
        XVec<BITS, BF16, CPL, GPC> xv;
        load_xvec<BITS, BF16, CPL, LPR, GPC>(xv, h + static_cast<int64_t>(r) * K, lane_in_row);
        const uint32_t *w = p.w + sl * p.w_slot;
        const uint16_t *s = p.s + sl * p.m_slot, *b = p.b + sl * p.m_slot;
        RowChunks<CPL> rc[J];
#pragma unroll
        for (int q = 0; q < J; ++q) {
            const int row = min(row0 + q * G::kRPL + row_sub, N - 1);
            load_row<BITS, CPL, LPR>(rc[q], w + row * wpr, lane_in_row);
        }
        float v[J];
#pragma unroll
        for (int q = 0; q < J; ++q) {
            const int row = min(row0 + q * G::kRPL + row_sub, N - 1);
            v[q] = row_partial<BITS, BF16, CPL, LPR, GPC>(rc[q], xv, s + row * gpr, b + row * gpr,
                                                          p.group, lane_in_row);
        }
        reduce_transposed<J, LPR>(v, lane);
        constexpr int span = LPR / J;
        const int vi = lane_in_row / span;
        if ((lane_in_row % span) == 0)
            ylds[j][vi * G::kRPL + row_sub] = valid_slot ? round16<BF16>(v[0]) : 0.f;
    }
    __syncthreads();
    for (int q = threadIdx.x; q < RPW; q += blockDim.x) {
        const int row = row0 + q;
        if (row >= N) continue;
        float acc = 0.f;
        for (int j = 0; j < ra.top_k; ++j) {
            const float w = round16<BF16>(ca.weights[t * ra.top_k + j]);
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
template <int BITS, bool BF16, int CPL, int LPR, int GPC>
hipError_t launch_gateup_t(const DecodeLaunch &L, hipStream_t st) {
    constexpr int J = 4;
    using G = Geom<BITS, CPL, LPR, GPC>;
    constexpr int waves = 4;
    const int rows_per_block = waves * J * G::kRPL;
    dim3 grid((L.gate.rows + rows_per_block - 1) / rows_per_block, L.routes);
    hipLaunchKernelGGL((gateup_route_kernel<BITS, BF16, CPL, LPR, GPC, J>), grid, dim3(64 * waves),
                       0, st, L.ra, L.gate, L.up, L.sgate, L.sup, L.h, L.limit, L.fp32_swiglu);
    return hipGetLastError();
}

template <int BITS, bool BF16, int CPL, int LPR, int GPC>
hipError_t launch_down_t(const DecodeLaunch &L, hipStream_t st) {
    constexpr int J = (LPR >= 8) ? 8 : LPR;
    using G = Geom<BITS, CPL, LPR, GPC>;
    const int rows_per_block = J * G::kRPL;
    const int per_token = L.ra.top_k + L.ra.n_shared;
    const int waves = per_token < kMaxRoutesPerToken ? per_token : kMaxRoutesPerToken;
    dim3 grid((L.down.rows + rows_per_block - 1) / rows_per_block, L.ra.tokens);
    hipLaunchKernelGGL((down_combine_kernel<BITS, BF16, CPL, LPR, GPC, J>), grid, dim3(64 * waves),
                       0, st, L.ra, L.down, L.sdown, L.h, L.ca);
    return hipGetLastError();
}

// which: 0 = gate/up, 1 = down+combine. (CPL, LPR) from 16-byte chunks per row.
template <int BITS, bool BF16, int GPC>
hipError_t decode_geometry(int which, int cpr, const DecodeLaunch &L, hipStream_t st) {
#define LOCALI_GEOM(CPL, LPR)                                                  \
    return which == 0 ? launch_gateup_t<BITS, BF16, CPL, LPR, GPC>(L, st)      \
                      : launch_down_t<BITS, BF16, CPL, LPR, GPC>(L, st)
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
