// Grouped expert kernels on the VALU: a tile is (slot, first sorted position,
// up to TT tokens). Every 32-bit weight word is expanded by v_and_or_b32 once
// and fed to TT v_dot2 instructions, one per token of the tile, so a slot's
// weights are streamed once per tile rather than once per route.
//
//   gateup_grouped_kernel  h[pos, n] = swiglu(gate, up) for the tile's tokens
//   down_grouped_kernel    y[pos, d] = round(down(h[pos]))
// Positions index the slot-sorted route order written by the dispatch; the
// shared expert's tile (slot marker -2) covers positions R .. R + tokens.
#pragma once

#include "launch.hpp"
#include "qgemv.hpp"

namespace locali {

struct TileArgs {
    const uint16_t *x;            // [tokens, d]
    const int32_t *tiles;         // [max_tiles, 4]
    const int32_t *n_tiles;       // [1]
    const int32_t *sorted_route;  // [R]
    int32_t R, top_k;
    int32_t n_vec;                // vectors in the MFMA kernels' input array (bounds of its loads)
    const int32_t *tile_tok;      // [max_tiles, 64] routed tiles' tokens by position (MFMA path)
    int32_t min_count;            // MFMA kernels: skip tiles of fewer positions (the small-tile kernels' share)
};

__device__ __forceinline__ int tile_token(const TileArgs &ta, bool shared, int pos) {
    return shared ? pos - ta.R : ta.sorted_route[pos] / ta.top_k;
}

// A routed tile of at most kPackedTokens positions carries its tokens in the
// tile record's last field: kTokensPacked, then kTokenBits bits per position
// (written by the dispatch; tokens below 2^kTokenBits).
constexpr int kPackedTokens = 2;
constexpr int kTokenBits = 15;
constexpr int32_t kTokensPacked = static_cast<int32_t>(0x40000000);

template <int BITS, bool BF16, int CPL, int LPR, int GPC, int TT>
__device__ __forceinline__ void row_partial_multi(const RowData<CPL, GPC> &rd,
                                                  const XVec<BITS, BF16, CPL, GPC> (&xv)[TT],
                                                  float (&out)[TT], uint32_t magic_v) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    using P = Pairs<BITS, BF16>;
#pragma unroll
    for (int q = 0; q < TT; ++q) out[q] = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const uint32_t words[4] = {rd.c[i][0], rd.c[i][1], rd.c[i][2], rd.c[i][3]};
#pragma unroll
        for (int gp = 0; gp < GPC; ++gp) {
            float d[TT];
#pragma unroll
            for (int q = 0; q < TT; ++q) d[q] = 0.f;
#pragma unroll
            for (int wd = gp * G::kWPG; wd < (gp + 1) * G::kWPG; ++wd) {
                static_for<0, P::kCount>([&](auto pc) {
                    constexpr int p = decltype(pc)::value;
                    const uint32_t a = expand_pair<BITS, BF16, p>(words[wd], magic_v);
#pragma unroll
                    for (int q = 0; q < TT; ++q) d[q] = dot2<BF16>(a, xv[q].xp[i][wd][p], d[q]);
                });
            }
            const float sc = to_float<BF16>(rd.s[i][gp]);
            const float bi = to_float<BF16>(rd.b[i][gp]);
#pragma unroll
            for (int q = 0; q < TT; ++q)
                out[q] = fmaf(sc, d[q] - xv[q].corr[i][gp], fmaf(bi, xv[q].xs[i][gp], out[q]));
        }
    }
}

constexpr int kGroupedWaves = 8;

// Prepare the tile's TT input vectors (rows of `src` selected by tile
// positions) into LDS; unused token slots repeat the last valid one.
template <int BITS, bool BF16, int CPL, int LPR, int TT, typename RowOf>
__device__ __forceinline__ void prep_tile(XLds<BITS, BF16, CPL, LPR> (&xl)[TT], RowOf row_of,
                                          int count) {
    constexpr int VPC = 128 / BITS, VPW = 32 / BITS;
    constexpr int units = LPR * CPL * 4;
    for (int u = threadIdx.x; u < TT * units; u += blockDim.x) {
        const int q = u / units, uu = u % units;
        const int ln = uu % LPR, wd = (uu / LPR) % 4, i = uu / (LPR * 4);
        const int k0 = (ln + LPR * i) * VPC + wd * VPW;
        prep_word<BITS, BF16>(row_of(min(q, count - 1)) + k0, &xl[q].pairs[i][wd][0][ln], LPR,
                              xl[q].part[i][wd][ln]);
    }
}

// SB: bits of the stored codes (BITS, or 3 for 3-bit rows widened to the
// 4-bit geometry on load).
template <int BITS, bool BF16, int CPL, int LPR, int GPC, int J, int TT, int SB = BITS>
__global__ __launch_bounds__(64 * kGroupedWaves) void gateup_grouped_kernel(
    TileArgs ta, QProj gate, QProj up, QProj sgate, QProj sup, uint16_t *__restrict__ h, float limit,
    int fp32_swiglu) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    constexpr int RPW = J * G::kRPL;
    constexpr int NV = 2 * J * TT;
    static_assert(NV <= LPR, "values per lane exceed lanes per row");
    __shared__ XLds<BITS, BF16, CPL, LPR> xl[TT];
    const int tile = blockIdx.y;
    if (tile >= *ta.n_tiles) return;
    const int slot = ta.tiles[4 * tile], first = ta.tiles[4 * tile + 1];
    const int count = ta.tiles[4 * tile + 2];
    const bool shared = slot == -2;
    // by value: the fields are selected in registers (a reference to one of
    // two parameter structs would make each field a dependent memory load)
    const QProj pg = shared ? sgate : gate;
    const QProj pu = shared ? sup : up;
    if (count <= 0 || (!shared && (slot < 0 || slot >= pg.n_slots || first < 0 ||
                                   first + count > ta.R)))
        return;
    const int N = pg.rows, K = pg.cols;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lane_in_row = lane % LPR, row_sub = lane / LPR;
    prep_tile<BITS, BF16, CPL, LPR, TT>(
        xl, [&](int q) { return ta.x + static_cast<int64_t>(tile_token(ta, shared, first + q)) * K; },
        count);
    __syncthreads();
    const int row0 = (blockIdx.x * (blockDim.x >> 6) + wave) * RPW;
    if (row0 >= N) return;
    const int sl = shared ? 0 : slot;
    const int64_t wpr = static_cast<int64_t>(K) * SB / 32;
    const int gpr = K / pg.group;
    const uint32_t *gw = pg.w + sl * pg.w_slot, *uw = pu.w + sl * pu.w_slot;
    const uint16_t *gs = pg.s + sl * pg.m_slot, *gb = pg.b + sl * pg.m_slot;
    const uint16_t *us = pu.s + sl * pu.m_slot, *ub = pu.b + sl * pu.m_slot;
    RowData<CPL, GPC> wg[J], wu[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int row = min(row0 + j * G::kRPL + row_sub, N - 1);
        load_row<BITS, CPL, LPR, GPC, SB>(wg[j], gw + row * wpr, gs + row * gpr, gb + row * gpr,
                                      pg.group, lane_in_row);
        load_row<BITS, CPL, LPR, GPC, SB>(wu[j], uw + row * wpr, us + row * gpr, ub + row * gpr,
                                      pu.group, lane_in_row);
    }
    XVec<BITS, BF16, CPL, GPC> xv[TT];
#pragma unroll
    for (int q = 0; q < TT; ++q) load_xvec_lds<BITS, BF16, CPL, LPR, GPC>(xv[q], xl[q], lane_in_row);
    sched_fence();
    const uint32_t magic_v = opaque_vgpr(Pairs<BITS, BF16>::kMagic);
    float v[NV];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        float pgq[TT], puq[TT];
        row_partial_multi<BITS, BF16, CPL, LPR, GPC, TT>(wg[j], xv, pgq, magic_v);
        row_partial_multi<BITS, BF16, CPL, LPR, GPC, TT>(wu[j], xv, puq, magic_v);
#pragma unroll
        for (int q = 0; q < TT; ++q) {
            v[j * TT + q] = pgq[q];
            v[J * TT + j * TT + q] = puq[q];
        }
    }
    reduce_transposed<NV, LPR>(v, lane);
    const float partner = shfl_xor(v[0], LPR / 2);
    constexpr int span = LPR / NV;
    const int vi = lane_in_row / span;
    if (vi < J * TT && (lane_in_row % span) == 0) {
        const int j = vi / TT, q = vi % TT;
        const int row = row0 + j * G::kRPL + row_sub;
        if (row < N && q < count)
            h[static_cast<int64_t>(first + q) * N + row] =
                swiglu16<BF16>(round16<BF16>(v[0]), round16<BF16>(partner), limit, fp32_swiglu != 0);
    }
}

template <int BITS, bool BF16, int CPL, int LPR, int GPC, int J, int TT, int SB = BITS>
__global__ __launch_bounds__(64 * kGroupedWaves) void down_grouped_kernel(
    TileArgs ta, QProj down, QProj sdown, const uint16_t *__restrict__ h, uint16_t *__restrict__ y) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    constexpr int RPW = J * G::kRPL;
    constexpr int NV = J * TT;
    static_assert(NV <= LPR, "values per lane exceed lanes per row");
    __shared__ XLds<BITS, BF16, CPL, LPR> xl[TT];
    const int tile = blockIdx.y;
    if (tile >= *ta.n_tiles) return;
    const int slot = ta.tiles[4 * tile], first = ta.tiles[4 * tile + 1];
    const int count = ta.tiles[4 * tile + 2];
    const bool shared = slot == -2;
    const QProj p = shared ? sdown : down;   // by value (see the gate/up kernel)
    if (count <= 0 || (!shared && (slot < 0 || slot >= p.n_slots || first < 0 ||
                                   first + count > ta.R)))
        return;
    const int N = p.rows, K = p.cols;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lane_in_row = lane % LPR, row_sub = lane / LPR;
    prep_tile<BITS, BF16, CPL, LPR, TT>(
        xl, [&](int q) { return h + static_cast<int64_t>(first + q) * K; }, count);
    __syncthreads();
    const int row0 = (blockIdx.x * (blockDim.x >> 6) + wave) * RPW;
    if (row0 >= N) return;
    const int sl = shared ? 0 : slot;
    const int64_t wpr = static_cast<int64_t>(K) * SB / 32;
    const int gpr = K / p.group;
    const uint32_t *w = p.w + sl * p.w_slot;
    const uint16_t *s = p.s + sl * p.m_slot, *b = p.b + sl * p.m_slot;
    RowData<CPL, GPC> rd[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int row = min(row0 + j * G::kRPL + row_sub, N - 1);
        load_row<BITS, CPL, LPR, GPC, SB>(rd[j], w + row * wpr, s + row * gpr, b + row * gpr, p.group,
                                      lane_in_row);
    }
    XVec<BITS, BF16, CPL, GPC> xv[TT];
#pragma unroll
    for (int q = 0; q < TT; ++q) load_xvec_lds<BITS, BF16, CPL, LPR, GPC>(xv[q], xl[q], lane_in_row);
    sched_fence();
    const uint32_t magic_v = opaque_vgpr(Pairs<BITS, BF16>::kMagic);
    float v[NV];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        float pq[TT];
        row_partial_multi<BITS, BF16, CPL, LPR, GPC, TT>(rd[j], xv, pq, magic_v);
#pragma unroll
        for (int q = 0; q < TT; ++q) v[j * TT + q] = pq[q];
    }
    reduce_transposed<NV, LPR>(v, lane);
    constexpr int span = LPR / NV;
    const int vi = lane_in_row / span;
    if ((lane_in_row % span) == 0) {
        const int j = vi / TT, q = vi % TT;
        const int row = row0 + j * G::kRPL + row_sub;
        if (row < N && q < count)
            y[static_cast<int64_t>(first + q) * N + row] = from_float<BF16>(v[0]);
    }
}

// --------------------------------------------------------------------------
constexpr int kGroupedTileTokens = 4;

struct GroupedKernelLaunch {
    TileArgs ta;
    bool bf16;
    QProj gate, up, down, sgate, sup, sdown;
    uint16_t *h, *y;
    float limit;
    int32_t fp32_swiglu;
    int32_t max_tiles;
};

template <int BITS, bool BF16, int CPL, int LPR, int GPC, int SB = BITS>
hipError_t launch_grouped_t(int which, const GroupedKernelLaunch &L, hipStream_t st) {
    constexpr int TT = kGroupedTileTokens;
    using G = Geom<BITS, CPL, LPR, GPC>;
    constexpr int waves = kGroupedWaves;
    if (which == 0) {
        constexpr int J = (LPR >= 4 * TT) ? 2 : 1;
        const int rpb = waves * J * G::kRPL;
        dim3 grid((L.gate.rows + rpb - 1) / rpb, L.max_tiles);
        hipLaunchKernelGGL((gateup_grouped_kernel<BITS, BF16, CPL, LPR, GPC, J, TT, SB>), grid,
                           dim3(64 * waves), 0, st, L.ta, L.gate, L.up, L.sgate, L.sup, L.h, L.limit,
                           L.fp32_swiglu);
    } else {
        constexpr int J = (LPR >= 4 * TT) ? 4 : ((LPR >= 2 * TT) ? 2 : 1);
        const int rpb = waves * J * G::kRPL;
        dim3 grid((L.down.rows + rpb - 1) / rpb, L.max_tiles);
        hipLaunchKernelGGL((down_grouped_kernel<BITS, BF16, CPL, LPR, GPC, J, TT, SB>), grid,
                           dim3(64 * waves), 0, st, L.ta, L.down, L.sdown, L.h, L.y);
    }
    return hipGetLastError();
}

template <int BITS, bool BF16, int GPC, int SB = BITS>
hipError_t grouped_geometry(int which, int cpr, const GroupedKernelLaunch &L, hipStream_t st) {
    switch (cpr) {
    case 8: return launch_grouped_t<BITS, BF16, 1, 8, GPC, SB>(which, L, st);
    case 16: return launch_grouped_t<BITS, BF16, 1, 16, GPC, SB>(which, L, st);
    case 32: return launch_grouped_t<BITS, BF16, 1, 32, GPC, SB>(which, L, st);
    case 64: return launch_grouped_t<BITS, BF16, 1, 64, GPC, SB>(which, L, st);
    case 128: return launch_grouped_t<BITS, BF16, 2, 64, GPC, SB>(which, L, st);
    case 256: return launch_grouped_t<BITS, BF16, 4, 64, GPC, SB>(which, L, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_grouped_kernels(int which, const GroupedKernelLaunch &L, hipStream_t st);

// The dispatch's placement step (stable sort of the routes by slot, see
// grouped.hip): its arguments, and its body for one 256-thread block (one
// wave per slot), shared by its own kernel and by the matrix-core path's
// fused place + input preparation launch.
struct PlaceArgs {
    const int32_t *route_slot;
    int R, n_slots;
    const int32_t *seg_start;
    int32_t *sorted_route, *route_pos;
    const int32_t *seg_tile;
    int32_t *tiles;
    int max_tiles, top_k, small_pack;
    int32_t *tile_tok;
    int tile_tokens;
};
constexpr int kPlaceSlotsPerBlock = 4;   // waves of a 256-thread block

__device__ __forceinline__ void dispatch_place_block(const PlaceArgs &a, int block) {
    const int lane = threadIdx.x & 63;
    const int s = block * kPlaceSlotsPerBlock + (threadIdx.x >> 6);
    if (s >= a.n_slots) return;
    const int base = a.seg_start[s], end = a.seg_start[s + 1];
    if (base == end) return;
    const int tile0 = a.seg_tile ? a.seg_tile[s] : -1;   // the segment's first tile
    // a slot of at most kPackedTokens routes: its tile's tokens, kTokenBits
    // bits each in position order, go into the tile record (see the count
    // kernel)
    int32_t *packed = nullptr;
    if (a.small_pack && end - base <= kPackedTokens && tile0 >= 0 && tile0 < a.max_tiles)
        packed = &a.tiles[4 * tile0 + 3];
    int32_t *tile_tok = tile0 < 0 ? nullptr : a.tile_tok;
    // 8 x 64 routes per pass: the loads of a pass are in flight together,
    // then the ballots place them in route order
    constexpr int U = 8;
    int pos = base;
    for (int r0 = 0; r0 < a.R && pos < end; r0 += 64 * U) {
        int v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = r0 + 64 * u + lane;
            v[u] = r < a.R ? a.route_slot[r] : -1;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int r = r0 + 64 * u + lane;
            const bool mine = v[u] == s;
            const uint64_t m = __ballot(mine);
            if (mine) {
                const int p = pos + __popcll(m & ((1ull << lane) - 1ull));
                a.sorted_route[p] = r;
                if (a.route_pos) a.route_pos[r] = p;
                if (packed) atomicOr(packed, (r / a.top_k) << (kTokenBits * (p - base)));
                if (tile_tok) {
                    const int q = p - base, tile = tile0 + q / a.tile_tokens;
                    if (tile < a.max_tiles)
                        tile_tok[static_cast<int64_t>(tile) * a.tile_tokens + q % a.tile_tokens] = r / a.top_k;
                }
            }
            pos += __popcll(m);
        }
    }
}

// The count step alone (one workgroup), filling `place` with the placement
// step's arguments (the caller launches it, possibly fused with other work).
hipError_t launch_dispatch_count(const int32_t *route_slot, int R, int n_slots, int n_shared_tokens,
                                 int tile_tokens, int32_t *seg_start, int32_t *sorted_route,
                                 int32_t *route_pos, int32_t *tiles, int32_t *n_tiles, int max_tiles,
                                 hipStream_t st, int32_t *seg_tile, int top_k, bool pack_small,
                                 int32_t *tile_tok, PlaceArgs *place);
hipError_t launch_dispatch(const int32_t *route_slot, int R, int n_slots, int n_shared_tokens,
                           int tile_tokens, int32_t *seg_start, int32_t *sorted_route,
                           int32_t *route_pos, int32_t *tiles, int32_t *n_tiles, int max_tiles,
                           hipStream_t st, int32_t *seg_tile = nullptr, int top_k = 0, bool pack_small = false,
                           int32_t *tile_tok = nullptr);
hipError_t launch_route_slots(const int32_t *idx, int R, int E, const int32_t *slot_of_expert,
                              int n_slots, int32_t *route_slot, hipStream_t st);
hipError_t launch_combine(const uint16_t *y, const int32_t *route_pos, const uint16_t *shared_y,
                          const float *weights, int tokens, int top_k, int d, int mode, bool bf16,
                          uint16_t *out, hipStream_t st);
hipError_t launch_combine_routes(const void *y, int y_type, const int32_t *route_pos,
                                 const uint16_t *shared_y, const float *weights, int tokens, int top_k,
                                 int d, int mode, bool bf16, uint16_t *out, hipStream_t st);

}  // namespace locali
