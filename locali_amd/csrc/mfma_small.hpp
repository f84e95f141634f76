// Grouped expert kernels for small tiles -- one or two positions of one slot
// for gate/up, one to four for down -- on the matrix cores (prefill, batched
// decode).
//
// The design of the decode gate/up kernel (mfma_decode.hpp): a wave owns a
// 512-value window of K for 32 rows, its 16-byte weight loads cover whole
// 128-byte lines, and the A operand is "diagonal". Its spare row bit carries
// the second position: A row m = 4 kb + 2 h + p holds position p's x' for
// k-lane kb's unit 4 h + kb, so D[4 kb + 2 h + p][n] is position p's dot with
// lane (n, kb)'s unit -- two positions for the MFMA work of one. For calls of
// many tokens the down stage takes tiles of up to four positions instead
// (down_small4_kernel: both pairs' MFMAs on each expanded weight register;
// measured 3.2 against the 64-position down kernel's 2.2 TB/s on such tiles,
// but slower than down_small_kernel on one- and two-position tiles, which
// dominate calls of few tokens; the gate/up kernel for three or four
// positions was slower than its 64-position kernel there). Under Zipf routing
// most experts of a prefill get one to four tokens; the tiles of the larger
// ones go to mfma_wide.hpp.
//
//   gateup_small_kernel  h[pos] = swiglu(up(x_t), gate(x_t)) for the tile's
//                        positions; x is prepared per wave in LDS; the epilogue
//                        writes h's prepared pairs (the MFMA layout) and sums
//                        per 32 values (the workgroup owns 32 rows).
//   down_small_kernel    y[pos] = round(down(h[pos])) for 32 output rows.
//   down_small4_kernel   the same for tiles of up to four positions.
// Reference arithmetic: dsv4_arena.py:168-235 (expert).
#pragma once

#include "mfma_decode.hpp"

namespace locali {

constexpr int kSmallGateUpTile = 2;   // positions of a small gate/up tile
constexpr int kSmallDownTile = 4;     // positions of a small down tile: one or two pairs
constexpr int kSmallRows = 32;  // rows per workgroup (2 tiles of 16)

struct SmallTileInfo {
    int slot, first, count, packed;
    bool shared;
};

// The tile's slot and positions, or false when this workgroup has nothing to
// do (past the list, a large tile, an invalid entry).
// The record and the tile count are read together: the grid has one row per
// possible tile, so the record is in bounds.
__device__ __forceinline__ bool small_tile(const TileArgs &ta, int tile, int n_slots, int max_count,
                                           SmallTileInfo &t) {
    const int4 rec = reinterpret_cast<const int4 *>(ta.tiles)[tile];
    const int nt = *ta.n_tiles;
    asm volatile("" ::"s"(rec.x), "s"(rec.y), "s"(rec.z), "s"(rec.w), "s"(nt));
    t.slot = rec.x;
    t.first = rec.y;
    t.count = rec.z;
    t.packed = rec.w;
    t.shared = t.slot == -2;
    if (tile >= nt || t.count <= 0 || t.count > max_count) return false;
    return t.shared || (t.slot >= 0 && t.slot < n_slots && t.first >= 0 && t.first + t.count <= ta.R);
}

// ---------------------------------------------------------------------------
template <int BITS, bool BF16>
__global__ __launch_bounds__(64 * kDiagGateUpMaxWaves) void gateup_small_kernel(
    TileArgs ta, QProj gate, QProj up, QProj sgate, QProj sup, MfmaVec hout, float2 *__restrict__ hsum32,
    int down_bits, float limit, int fp32_swiglu) {
    using G = DiagGeom<BITS>;
    constexpr int RT = kSmallRows / 16;
    constexpr int NI = 2 * G::kLines;
    __shared__ __align__(16) DiagSlice<BITS> win[kDiagGateUpMaxWaves][kSmallGateUpTile];
    __shared__ float red[kDiagGateUpMaxWaves][RT][2][kSmallGateUpTile][16];
    __shared__ __align__(16) uint16_t hs[kSmallGateUpTile][kSmallRows];
    __shared__ __align__(16) uint8_t mlds[4 * kSmallRows * (2 * (4096 / 64) + 16)];
    SmallTileInfo ti;
    if (!small_tile(ta, blockIdx.y, gate.n_slots, kSmallGateUpTile, ti)) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nl = lane & 15, kb = lane >> 4, hh = nl >> 3, r8 = nl & 7;
    const bool shared = ti.shared;
    const int sl = shared ? 0 : ti.slot, count = ti.count;
    const int N = gate.rows, K = gate.cols;
    const uint32_t *gwp = shared ? sgate.w : gate.w, *uwp = shared ? sup.w : up.w;
    const int64_t gw_slot = shared ? sgate.w_slot : gate.w_slot, uw_slot = shared ? sup.w_slot : up.w_slot;
    const int64_t gm_slot = shared ? sgate.m_slot : gate.m_slot, um_slot = shared ? sup.m_slot : up.m_slot;
    const int n0 = blockIdx.x * kSmallRows;
    const int wpr = K * BITS / 32, gpr = K / gate.group;
    const int waves = blockDim.x >> 6;   // = K / 512
    const int ug_log2 = units_per_group_log2<BITS>(gate.group);
    // tokens from the tile record when the dispatch packed them there
    static_assert(kSmallGateUpTile <= kPackedTokens, "small tiles carry packed tokens");
    const bool packed = !shared && (ti.packed & kTokensPacked);
    int tok[kSmallGateUpTile];
#pragma unroll
    for (int p = 0; p < kSmallGateUpTile; ++p) {
        const int q = min(p, count - 1);
        tok[p] = packed ? (ti.packed >> (kTokenBits * q)) & ((1 << kTokenBits) - 1)
                        : tile_token(ta, shared, ti.first + q);
    }

    // Raw x of the window of each position, the workgroup's scales and biases
    // by whole lines, then the weights in consumption order.
    uint32_t xw[kSmallGateUpTile][16 / BITS];
#pragma unroll
    for (int p = 0; p < kSmallGateUpTile; ++p)
        diag_prep_load<BITS>(xw[p], ta.x + static_cast<int64_t>(tok[p]) * K + wave * kDiagWindow, lane);
    sched_fence();
    const int mrs = 2 * gpr + 16;
    const int64_t mrow0 = static_cast<int64_t>(n0) * gpr;
    const uint16_t *m_gs = (shared ? sgate.s : gate.s) + sl * gm_slot + mrow0;
    const uint16_t *m_gb = (shared ? sgate.b : gate.b) + sl * gm_slot + mrow0;
    const uint16_t *m_us = (shared ? sup.s : up.s) + sl * um_slot + mrow0;
    const uint16_t *m_ub = (shared ? sup.b : up.b) + sl * um_slot + mrow0;
    u32x4 mv0, mv1;
    const MetaPiece mp0 = meta_piece_of(static_cast<int>(threadIdx.x), 4, kSmallRows, gpr, mrs);
    const MetaPiece mp1 = meta_piece_of(static_cast<int>(threadIdx.x) + 64 * waves, 4, kSmallRows, gpr, mrs);
    auto meta_load = [&](const MetaPiece &m) {
        const uint16_t *arr = m.arr == 0 ? m_gs : m.arr == 1 ? m_gb : m.arr == 2 ? m_us : m_ub;
        return *reinterpret_cast<const u32x4 *>(arr + m.off);
    };
    mv0 = meta_load(mp0);
    mv1 = meta_load(mp1);
    sched_fence();
    const uint32_t wbytes = 4u * kSmallRows * wpr;
    const int64_t wrow0 = static_cast<int64_t>(n0) * wpr;
    const __amdgpu_buffer_rsrc_t gw_rs = make_rsrc(gwp + sl * gw_slot + wrow0, wbytes);
    const __amdgpu_buffer_rsrc_t uw_rs = make_rsrc(uwp + sl * uw_slot + wrow0, wbytes);
    u32x4 wg[RT][NI], wu[RT][NI];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int q = 0; q < NI; ++q) {
            const int i = q & 1, line = q >> 1;
            const uint32_t wo = 4u * static_cast<uint32_t>((16 * rt + 8 * i + r8) * wpr) + 128u * line +
                                16u * (4 * hh + kb);
            wg[rt][q] = __builtin_amdgcn_raw_buffer_load_b128(gw_rs, wo, 128 * G::kLines * wave, kAuxStream);
            wu[rt][q] = __builtin_amdgcn_raw_buffer_load_b128(uw_rs, wo, 128 * G::kLines * wave, kAuxStream);
        }
    sched_fence();
    diag_prep_store<BITS, BF16>(win[wave][0], xw[0], lane);
    if (count > 1) diag_prep_store<BITS, BF16>(win[wave][1], xw[1], lane);
    if (mp0.store) *reinterpret_cast<u32x4 *>(mlds + mp0.dst) = mv0;
    if (mp1.store) *reinterpret_cast<u32x4 *>(mlds + mp1.dst) = mv1;
    __syncthreads();
    const uint32_t magic_v = opaque_vgpr(Pairs<BITS, BF16>::kMagic);
    // A lane (m, kb) feeds position m % 2's unit 8 line + 4 ((m / 2) % 2) + kb when m / 4 == kb
    const int ap = nl & 1;
    const bool feed = (nl >> 2) == kb && ap < count;
    const int ah = (nl >> 1) & 1;
    const int as = kSmallRows * mrs / 2;
    float accg[RT][2][kSmallGateUpTile], accu[RT][2][kSmallGateUpTile];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < kSmallGateUpTile; ++p) accg[rt][i][p] = accu[rt][i][p] = 0.f;
#pragma unroll
    for (int line = 0; line < G::kLines; ++line) {
        const int uA = 8 * line + 4 * ah + kb;
        const uint8_t *abase = feed ? win[wave][ap].pairs + uA * G::kStride
                                    : reinterpret_cast<const uint8_t *>(win[wave][0].zero);
        mf32x4_t dg[RT][2], du[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                dg[rt][i] = mf32x4_t{0.f, 0.f, 0.f, 0.f};
                du[rt][i] = dg[rt][i];
            }
        static_for<0, G::kSteps>([&](auto tc) {
            constexpr int t = decltype(tc)::value;
            const u32x4 a = reinterpret_cast<const u32x4 *>(abase)[t];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    dg[rt][i] = mfma_16x16x32<BF16>(a, diag_b<BITS, BF16, t>(wg[rt][2 * line + i], magic_v),
                                                    dg[rt][i]);
                    du[rt][i] = mfma_16x16x32<BF16>(a, diag_b<BITS, BF16, t>(wu[rt][2 * line + i], magic_v),
                                                    du[rt][i]);
                }
        });
        const int uB = 8 * line + 4 * hh + kb;
        const float2 us0 = win[wave][0].usum[uB];
        const float2 us1 = win[wave][1].usum[uB];
        const int grp = (G::kUnits * wave + uB) >> ug_log2;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint16_t *m0 = reinterpret_cast<const uint16_t *>(mlds + (16 * rt + 8 * i + r8) * mrs) + grp;
                const uint16_t s_g = m0[0], b_g = m0[as], s_u = m0[2 * as], b_u = m0[3 * as];
                accg[rt][i][0] += diag_fix<BF16>(hh ? dg[rt][i][2] : dg[rt][i][0], s_g, b_g, us0);
                accu[rt][i][0] += diag_fix<BF16>(hh ? du[rt][i][2] : du[rt][i][0], s_u, b_u, us0);
                accg[rt][i][1] += diag_fix<BF16>(hh ? dg[rt][i][3] : dg[rt][i][1], s_g, b_g, us1);
                accu[rt][i][1] += diag_fix<BF16>(hh ? du[rt][i][3] : du[rt][i][1], s_u, b_u, us1);
            }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < kSmallGateUpTile; ++p) {
                const float g = diag_row_sum(accg[rt][i][p]);
                const float u = diag_row_sum(accu[rt][i][p]);
                if (lane < 8) {
                    red[wave][rt][0][p][8 * i + lane] = g;
                    red[wave][rt][1][p][8 * i + lane] = u;
                }
            }
    __syncthreads();
    if (wave != 0) return;
    // Wave 0: h of the tile's positions in window order, then h's prepared
    // form: pairs and the sum of each position's 32 values.
    if (lane < kSmallRows * count) {
        const int p = lane / kSmallRows, q = lane % kSmallRows, rt = q >> 4, n = q & 15;
        float g = 0.f, u = 0.f;
        for (int w = 0; w < waves; ++w) {
            g += red[w][rt][0][p][n];
            u += red[w][rt][1][p][n];
        }
        hs[p][q] = swiglu16<BF16>(round16<BF16>(g), round16<BF16>(u), limit, fp32_swiglu != 0);
        if (hout.plain) hout.plain[static_cast<int64_t>(ti.first + p) * N + n0 + q] = hs[p][q];
    }
    const int vpw = 32 / down_bits, words = kSmallRows / vpw;
    float2 part = make_float2(0.f, 0.f);
    const int p = lane / words, wi = lane % words;
    if (lane < words * count)
        prep_unit_at<BF16>(down_bits, &hs[p][wi * vpw],
                           hout.pairs + (ti.first + p) * hout.pairs_stride +
                               (n0 / vpw + wi) * pairs_per_word<BF16>(down_bits),
                           &part);
    for (int m = 1; m < words; m <<= 1) {
        part.x += __shfl_xor(part.x, m, 64);
        part.y += __shfl_xor(part.y, m, 64);
    }
    if (lane < words * count && wi == 0) hsum32[static_cast<int64_t>(ti.first + p) * (N / 32) + n0 / 32] = part;
}

// ---------------------------------------------------------------------------
template <int BITS, bool BF16>
__global__ __launch_bounds__(64 * kDiagGateUpMaxWaves) void down_small_kernel(
    TileArgs ta, QProj down, QProj sdown, MfmaVec hin, const float2 *__restrict__ hsum32,
    uint16_t *__restrict__ y) {
    using G = DiagGeom<BITS>;
    constexpr int RT = kSmallRows / 16;
    constexpr int NI = 2 * G::kLines;
    __shared__ __align__(16) DiagSlice<BITS> win[kDiagGateUpMaxWaves][kSmallGateUpTile];
    __shared__ float red[kDiagGateUpMaxWaves][RT][kSmallGateUpTile][16];
    __shared__ __align__(16) uint8_t mlds[2 * kSmallRows * (2 * (4096 / 64) + 16)];
    SmallTileInfo ti;
    if (!small_tile(ta, blockIdx.y, down.n_slots, kSmallGateUpTile, ti)) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nl = lane & 15, kb = lane >> 4, hh = nl >> 3, r8 = nl & 7;
    const bool shared = ti.shared;
    const int sl = shared ? 0 : ti.slot, count = ti.count;
    const int N = down.rows, K = down.cols;
    const uint32_t *wp = shared ? sdown.w : down.w;
    const int64_t w_slot = shared ? sdown.w_slot : down.w_slot, m_slot = shared ? sdown.m_slot : down.m_slot;
    const int n0 = blockIdx.x * kSmallRows;
    const int wpr = K * BITS / 32, gpr = K / down.group;
    const int waves = blockDim.x >> 6;   // = K / 512
    const int ug_log2 = units_per_group_log2<BITS>(down.group);

    // The window's prepared h of each position and the sums of the lane's
    // units (a 64-value unit adds its two 32-value halves), the scales and
    // biases by whole lines, then the weights.
    u32x4 hv[kSmallGateUpTile];
    float2 hsum[kSmallGateUpTile][G::kLines];
#pragma unroll
    for (int p = 0; p < kSmallGateUpTile; ++p) {
        const int pos = ti.first + min(p, count - 1);
        hv[p] = reinterpret_cast<const u32x4 *>(hin.pairs + pos * hin.pairs_stride + wave * (kDiagWindow / 2))[lane];
#pragma unroll
        for (int line = 0; line < G::kLines; ++line) {
            const int u = G::kUnits * wave + 8 * line + 4 * hh + kb;   // unit of K
            const float2 *hp = hsum32 + static_cast<int64_t>(pos) * (K / 32) + u * (G::kUnitVals / 32);
            if constexpr (G::kUnitVals == 64) {
                const float4 s2 = reinterpret_cast<const float4 *>(hp)[0];
                hsum[p][line] = make_float2(s2.x + s2.z, s2.y + s2.w);
            } else {
                hsum[p][line] = hp[0];
            }
        }
    }
    sched_fence();
    const int mrs = 2 * gpr + 16;
    const int64_t mrow0 = static_cast<int64_t>(n0) * gpr;
    const uint16_t *m_s = (shared ? sdown.s : down.s) + sl * m_slot + mrow0;
    const uint16_t *m_b = (shared ? sdown.b : down.b) + sl * m_slot + mrow0;
    // 2 arrays x 32 rows x gpr / 8 pieces: at most one per thread
    const MetaPiece mp = meta_piece_of(static_cast<int>(threadIdx.x), 2, kSmallRows, gpr, mrs);
    const u32x4 mv = *reinterpret_cast<const u32x4 *>((mp.arr == 0 ? m_s : m_b) + mp.off);
    sched_fence();
    const __amdgpu_buffer_rsrc_t w_rs =
        make_rsrc(wp + sl * w_slot + static_cast<int64_t>(n0) * wpr, 4u * kSmallRows * wpr);
    u32x4 wd[RT][NI];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int q = 0; q < NI; ++q) {
            const int i = q & 1, line = q >> 1;
            const uint32_t wo = 4u * static_cast<uint32_t>((16 * rt + 8 * i + r8) * wpr) + 128u * line +
                                16u * (4 * hh + kb);
            wd[rt][q] = __builtin_amdgcn_raw_buffer_load_b128(w_rs, wo, 128 * G::kLines * wave, kAuxStream);
        }
    sched_fence();
    {
        constexpr int LPU = G::kUnitPairs / 4;   // lanes per unit
#pragma unroll
        for (int p = 0; p < kSmallGateUpTile; ++p)
            *reinterpret_cast<u32x4 *>(win[wave][p].pairs + (lane / LPU) * G::kStride + 16 * (lane % LPU)) = hv[p];
        if (lane < 4 * G::kSteps) win[wave][0].zero[lane] = 0u;
    }
    if (mp.store) *reinterpret_cast<u32x4 *>(mlds + mp.dst) = mv;
    __syncthreads();
    const uint32_t magic_v = opaque_vgpr(Pairs<BITS, BF16>::kMagic);
    const int ap = nl & 1;
    const bool feed = (nl >> 2) == kb && ap < count;
    const int ah = (nl >> 1) & 1;
    const int as = kSmallRows * mrs / 2;
    float acc[RT][2][kSmallGateUpTile];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < kSmallGateUpTile; ++p) acc[rt][i][p] = 0.f;
#pragma unroll
    for (int line = 0; line < G::kLines; ++line) {
        const int uA = 8 * line + 4 * ah + kb;
        const uint8_t *abase = feed ? win[wave][ap].pairs + uA * G::kStride
                                    : reinterpret_cast<const uint8_t *>(win[wave][0].zero);
        mf32x4_t d[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < 2; ++i) d[rt][i] = mf32x4_t{0.f, 0.f, 0.f, 0.f};
        static_for<0, G::kSteps>([&](auto tc) {
            constexpr int t = decltype(tc)::value;
            const u32x4 a = reinterpret_cast<const u32x4 *>(abase)[t];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    d[rt][i] = mfma_16x16x32<BF16>(a, diag_b<BITS, BF16, t>(wd[rt][2 * line + i], magic_v), d[rt][i]);
        });
        const int uB = 8 * line + 4 * hh + kb;
        const int grp = (G::kUnits * wave + uB) >> ug_log2;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint16_t *m0 = reinterpret_cast<const uint16_t *>(mlds + (16 * rt + 8 * i + r8) * mrs) + grp;
                const uint16_t s = m0[0], b = m0[as];
                acc[rt][i][0] += diag_fix<BF16>(hh ? d[rt][i][2] : d[rt][i][0], s, b, hsum[0][line]);
                acc[rt][i][1] += diag_fix<BF16>(hh ? d[rt][i][3] : d[rt][i][1], s, b, hsum[1][line]);
            }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int p = 0; p < kSmallGateUpTile; ++p) {
                const float v = diag_row_sum(acc[rt][i][p]);
                if (lane < 8) red[wave][rt][p][8 * i + lane] = v;
            }
    __syncthreads();
    if (wave != 0 || lane >= kSmallRows * count) return;
    const int p = lane / kSmallRows, q = lane % kSmallRows, rt = q >> 4, n = q & 15;
    float v = 0.f;
    for (int w = 0; w < waves; ++w) v += red[w][rt][p][n];
    y[static_cast<int64_t>(ti.first + p) * N + n0 + q] = from_float<BF16>(v);
}


template <int BITS, bool BF16>
__global__ __launch_bounds__(64 * kDiagGateUpMaxWaves) void down_small4_kernel(
    TileArgs ta, QProj down, QProj sdown, MfmaVec hin, const float2 *__restrict__ hsum32,
    uint16_t *__restrict__ y) {
    using G = DiagGeom<BITS>;
    constexpr int RT = kSmallRows / 16;
    constexpr int NI = 2 * G::kLines;
    extern __shared__ __align__(16) uint8_t small_win[];
    auto win = reinterpret_cast<DiagSlice<BITS>(*)[kSmallDownTile]>(small_win);
    __shared__ float red[kDiagGateUpMaxWaves][RT][kSmallDownTile][16];
    __shared__ __align__(16) uint8_t mlds[2 * kSmallRows * (2 * (4096 / 64) + 16)];
    SmallTileInfo ti;
    if (!small_tile(ta, blockIdx.y, down.n_slots, kSmallDownTile, ti)) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nl = lane & 15, kb = lane >> 4, hh = nl >> 3, r8 = nl & 7;
    const bool shared = ti.shared;
    const int sl = shared ? 0 : ti.slot, count = ti.count;
    const int N = down.rows, K = down.cols;
    const uint32_t *wp = shared ? sdown.w : down.w;
    const int64_t w_slot = shared ? sdown.w_slot : down.w_slot, m_slot = shared ? sdown.m_slot : down.m_slot;
    const int n0 = blockIdx.x * kSmallRows;
    const int wpr = K * BITS / 32, gpr = K / down.group;
    const int waves = blockDim.x >> 6;   // = K / 512
    const int ug_log2 = units_per_group_log2<BITS>(down.group);

    // The window's prepared h of each position and the sums of the lane's
    // units (a 64-value unit adds its two 32-value halves), the scales and
    // biases by whole lines, then the weights.
    u32x4 hv[kSmallDownTile];
    float2 hsum[kSmallDownTile][G::kLines];
#pragma unroll
    for (int p = 0; p < kSmallDownTile; ++p) {
        const int pos = ti.first + min(p, count - 1);
        hv[p] = reinterpret_cast<const u32x4 *>(hin.pairs + pos * hin.pairs_stride + wave * (kDiagWindow / 2))[lane];
#pragma unroll
        for (int line = 0; line < G::kLines; ++line) {
            const int u = G::kUnits * wave + 8 * line + 4 * hh + kb;   // unit of K
            const float2 *hp = hsum32 + static_cast<int64_t>(pos) * (K / 32) + u * (G::kUnitVals / 32);
            if constexpr (G::kUnitVals == 64) {
                const float4 s2 = reinterpret_cast<const float4 *>(hp)[0];
                hsum[p][line] = make_float2(s2.x + s2.z, s2.y + s2.w);
            } else {
                hsum[p][line] = hp[0];
            }
        }
    }
    sched_fence();
    const int mrs = 2 * gpr + 16;
    const int64_t mrow0 = static_cast<int64_t>(n0) * gpr;
    const uint16_t *m_s = (shared ? sdown.s : down.s) + sl * m_slot + mrow0;
    const uint16_t *m_b = (shared ? sdown.b : down.b) + sl * m_slot + mrow0;
    // 2 arrays x 32 rows x gpr / 8 pieces: at most one per thread
    const MetaPiece mp = meta_piece_of(static_cast<int>(threadIdx.x), 2, kSmallRows, gpr, mrs);
    const u32x4 mv = *reinterpret_cast<const u32x4 *>((mp.arr == 0 ? m_s : m_b) + mp.off);
    sched_fence();
    const __amdgpu_buffer_rsrc_t w_rs =
        make_rsrc(wp + sl * w_slot + static_cast<int64_t>(n0) * wpr, 4u * kSmallRows * wpr);
    u32x4 wd[RT][NI];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int q = 0; q < NI; ++q) {
            const int i = q & 1, line = q >> 1;
            const uint32_t wo = 4u * static_cast<uint32_t>((16 * rt + 8 * i + r8) * wpr) + 128u * line +
                                16u * (4 * hh + kb);
            wd[rt][q] = __builtin_amdgcn_raw_buffer_load_b128(w_rs, wo, 128 * G::kLines * wave, kAuxStream);
        }
    sched_fence();
    {
        constexpr int LPU = G::kUnitPairs / 4;   // lanes per unit
#pragma unroll
        for (int p = 0; p < kSmallDownTile; ++p)
            *reinterpret_cast<u32x4 *>(win[wave][p].pairs + (lane / LPU) * G::kStride + 16 * (lane % LPU)) = hv[p];
        if (lane < 4 * G::kSteps) win[wave][0].zero[lane] = 0u;
    }
    if (mp.store) *reinterpret_cast<u32x4 *>(mlds + mp.dst) = mv;
    __syncthreads();
    const int ap = nl & 1;
    const int ah = (nl >> 1) & 1;
    const int as = kSmallRows * mrs / 2;
    auto compute = [&](auto npc) {
        constexpr int NPR = decltype(npc)::value;   // position pairs
        const uint32_t magic_v = opaque_vgpr(Pairs<BITS, BF16>::kMagic);
        bool feed[NPR];
#pragma unroll
        for (int pr = 0; pr < NPR; ++pr) feed[pr] = (nl >> 2) == kb && 2 * pr + ap < count;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float acc[2][2 * NPR];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int p = 0; p < 2 * NPR; ++p) acc[i][p] = 0.f;
#pragma unroll
            for (int line = 0; line < G::kLines; ++line) {
                const int uA = 8 * line + 4 * ah + kb;
                const uint8_t *abase[NPR];
#pragma unroll
                for (int pr = 0; pr < NPR; ++pr)
                    abase[pr] = feed[pr] ? win[wave][2 * pr + ap].pairs + uA * G::kStride
                                         : reinterpret_cast<const uint8_t *>(win[wave][0].zero);
                mf32x4_t d[NPR][2];
#pragma unroll
                for (int pr = 0; pr < NPR; ++pr)
#pragma unroll
                    for (int i = 0; i < 2; ++i) d[pr][i] = mf32x4_t{0.f, 0.f, 0.f, 0.f};
                static_for<0, G::kSteps>([&](auto tc) {
                    constexpr int t = decltype(tc)::value;
                    u32x4 a[NPR];
#pragma unroll
                    for (int pr = 0; pr < NPR; ++pr) a[pr] = reinterpret_cast<const u32x4 *>(abase[pr])[t];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const u32x4 b = diag_b<BITS, BF16, t>(wd[rt][2 * line + i], magic_v);
#pragma unroll
                        for (int pr = 0; pr < NPR; ++pr) d[pr][i] = mfma_16x16x32<BF16>(a[pr], b, d[pr][i]);
                    }
                });
                const int uB = 8 * line + 4 * hh + kb;
                const int grp = (G::kUnits * wave + uB) >> ug_log2;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint16_t *m0 =
                        reinterpret_cast<const uint16_t *>(mlds + (16 * rt + 8 * i + r8) * mrs) + grp;
                    const uint16_t s = m0[0], b = m0[as];
#pragma unroll
                    for (int pr = 0; pr < NPR; ++pr) {
                        acc[i][2 * pr] += diag_fix<BF16>(hh ? d[pr][i][2] : d[pr][i][0], s, b, hsum[2 * pr][line]);
                        acc[i][2 * pr + 1] +=
                            diag_fix<BF16>(hh ? d[pr][i][3] : d[pr][i][1], s, b, hsum[2 * pr + 1][line]);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int p = 0; p < 2 * NPR; ++p) {
                    const float v = diag_row_sum(acc[i][p]);
                    if (lane < 8) red[wave][rt][p][8 * i + lane] = v;
                }
        }
    };
    if (count > 2)
        compute(std::integral_constant<int, 2>{});
    else
        compute(std::integral_constant<int, 1>{});
    __syncthreads();
    if (wave != 0) return;
    for (int e = lane; e < kSmallRows * count; e += 64) {
        const int p = e / kSmallRows, q = e % kSmallRows, rt = q >> 4, n = q & 15;
        float v = 0.f;
        for (int w = 0; w < waves; ++w) v += red[w][rt][p][n];
        y[static_cast<int64_t>(ti.first + p) * N + n0 + q] = from_float<BF16>(v);
    }
}

// The four-position down kernel's windows in dynamic LDS at the most waves
// (K = 4096).
template <int BITS>
constexpr size_t kSmallDownMaxWinLds = kDiagGateUpMaxWaves * kSmallDownTile * sizeof(DiagSlice<BITS>);

// which: 3 = gate/up of small tiles, 4 = down of small tiles (of up to
// L.small_down_positions positions: 2 or kSmallDownTile).
template <int BITS, bool BF16>
hipError_t launch_small_stage(int which, const MfmaLaunch &L, hipStream_t st) {
    TileArgs ta = L.ta;
    if (which == 3) {
        dim3 grid(L.gate.rows / kSmallRows, L.max_tiles);
        hipLaunchKernelGGL((gateup_small_kernel<BITS, BF16>), grid, dim3(64 * (L.gate.cols / kDiagWindow)), 0, st,
                           ta, L.gate, L.up, L.sgate, L.sup, L.hmid, L.hsum32, L.down.bits, L.limit,
                           L.fp32_swiglu);
    } else if (L.small_down_positions == kSmallDownTile) {
        dim3 grid(L.down.rows / kSmallRows, L.max_tiles);
        const int waves = L.down.cols / kDiagWindow;
        const size_t lds = waves * kSmallDownTile * sizeof(DiagSlice<BITS>);
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&down_small4_kernel<BITS, BF16>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kSmallDownMaxWinLds<BITS>));
        if (attr != hipSuccess) return attr;
        hipLaunchKernelGGL((down_small4_kernel<BITS, BF16>), grid, dim3(64 * waves), lds, st, ta, L.down, L.sdown,
                           L.hmid, L.hsum32, L.y);
    } else {
        dim3 grid(L.down.rows / kSmallRows, L.max_tiles);
        hipLaunchKernelGGL((down_small_kernel<BITS, BF16>), grid, dim3(64 * (L.down.cols / kDiagWindow)), 0, st,
                           ta, L.down, L.sdown, L.hmid, L.hsum32, L.y);
    }
    return hipGetLastError();
}

}  // namespace locali
