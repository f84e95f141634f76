// Decode-path gate/up kernel on the matrix cores (one token per route).
//
// A wave owns 16 output rows (a row tile) and a 512-value window of K. Its
// weight loads cover whole 128-byte lines: in one 16-byte load, lane (n =
// lane % 16, kb = lane / 16) reads "unit" 4 h + kb (h = n / 8) of the line of
// row 8 i + n % 8, so 8 lanes read a row's line and one load covers 8 rows.
// A unit is 16 bytes of codes: one 64-value block at 2 bits, half a block at
// 4 bits. Every MFMA step (v_mfma_f32_16x16x32) takes 8 values of the lane's
// unit from each k-lane; the A operand is "diagonal": A[m][k] holds x' of
// k-lane kb(k)'s unit 4 h + kb only in rows m with m / 4 == kb and
// (m / 2) % 2 == h, zero elsewhere, so D[4 kb + 2 h][n] is exactly the dot of
// lane (n, kb)'s unit with x -- the product keeps the units apart and every
// lane receives its own unit's dot. The per-unit affine terms
//   acc += s * (D - magic * sum x') + b * sum x        (dsv4_kernels.py:75-79)
// are one instruction each for 64 (row, unit) pairs, and the units of a row
// meet by three cross-lane adds. The zero rows of A come from a zeroed LDS
// slot read by the off-diagonal lanes, so building A costs LDS reads, not
// VALU; the VALU is left with the dequant (one v_bitop3_b32 per value pair)
// and the matrix core does every product.
//
//   gateup_diag_kernel  h[r, n] = swiglu(up_r(x_t)[n], gate_r(x_t)[n]): a
//                       workgroup is 32 rows of one route, one wave per
//                       window of K (K / 512 waves). Each wave prepares its
//                       window of x into its own LDS slice while the weights
//                       stream in; the workgroup's scales and biases arrive
//                       by whole lines into LDS; the windows meet in LDS in
//                       window order. The epilogue writes h and its prepared
//                       form (pairs and per-word sums, the decode layout: the
//                       workgroup owns whole words of the down input).
// The down projection and combine of the decode path stay on the VALU
// kernel (decode_kernels.hpp), which reads the same hidden layout.
// Reference arithmetic: dsv4_arena.py:168-235 (expert).
#pragma once

#include "decode_kernels.hpp"
#include "mfma_grouped.hpp"
#include "router_select.hpp"

namespace locali {

// 3-bit gate/up rows staged in LDS: a 192-byte window row padded to 52
// words, one 16-row tile a wave at a time
constexpr int kDiag3RowWords = 52;
constexpr size_t kDiag3WaveBytes = 4 * kDiag3RowWords * 16;

template <int BITS>
struct DiagGeom {
    // BITS: the width the kernels compute in (3-bit codes are widened to 4)
    static constexpr int kUnitVals = 128 / BITS;            // values per 16-byte unit
    static constexpr int kUnits = kDiagWindow / kUnitVals;  // units per window row (8 or 16)
    static constexpr int kLines = kUnits / 8;               // 128-byte lines per window row
    static constexpr int kSteps = kUnitVals / 8;            // MFMA steps per unit
    static constexpr int kUnitPairs = kUnitVals / 2;        // prepared pairs per unit
    static constexpr int kStride = 4 * kUnitPairs + 16;     // LDS bytes per unit (padded)
    static constexpr int kUnitsPerGroup = 64 / kUnitVals;   // group 64
    static_assert(BITS == 2 || BITS == 4, "2- and 4-bit codes");
};

// A workgroup's scales and biases (`arrays` arrays of `rows` rows of gpr
// groups) move into LDS by whole lines as 16-byte pieces: piece c = (array,
// row, part), gpr / 8 parts per row, row stride mrs bytes in LDS. With
// groups of 128 there are half as many pieces as with 64; a thread whose
// piece lies past the arrays loads a valid piece again (the loads stay
// unconditional, so the vector-memory counter keeps counting them) and does
// not store it.
struct MetaPiece {
    int arr;      // array index (clamped)
    int off;      // u16 offset in the array's rows
    int dst;      // LDS byte offset
    bool store;
};

__device__ __forceinline__ MetaPiece meta_piece_of(int c, int arrays, int rows, int gpr, int mrs) {
    const int ppr = gpr >> 3;
    const int a = c / (rows * ppr), row = (c / ppr) % rows, pc = c % ppr;
    MetaPiece m;
    m.store = a < arrays;
    m.arr = min(a, arrays - 1);
    m.off = row * gpr + 8 * pc;
    m.dst = (a * rows + row) * mrs + 16 * pc;
    return m;
}

// log2 of the 16-byte units a group of `group` values spans (groups of 64
// or 128): grp = unit >> units_per_group_log2.
template <int BITS>
__device__ __forceinline__ int units_per_group_log2(int group) {
    constexpr int base = DiagGeom<BITS>::kUnitsPerGroup == 1 ? 0 : DiagGeom<BITS>::kUnitsPerGroup == 2 ? 1 : 2;
    return base + (group == 128 ? 1 : 0);
}

// One window of a prepared vector in LDS: unit u's pairs at u * kStride
// (padding spreads the eight units one step reads over distinct banks), then
// a zeroed slot for the off-diagonal lanes, then the per-unit sums
// (magic * sum x', sum x).
template <int BITS>
struct DiagSlice {
    using G = DiagGeom<BITS>;
    uint8_t pairs[G::kUnits * G::kStride];
    uint32_t zero[4 * G::kSteps];
    float2 usum[G::kUnits];
};

// Raw values of the lane's word of a window (lanes past the window's words
// read the last word again; their values are not used).
template <int BITS>
__device__ __forceinline__ void diag_prep_load(uint32_t (&ww)[16 / BITS], const uint16_t *win_src, int lane) {
    constexpr int VPW = 32 / BITS, WORDS = kDiagWindow / VPW;
    const uint4 *p = reinterpret_cast<const uint4 *>(win_src + min(lane, WORDS - 1) * VPW);
    if constexpr (BITS == 2) {
        const uint4 a = p[0], c = p[1];
        ww[0] = a.x; ww[1] = a.y; ww[2] = a.z; ww[3] = a.w;
        ww[4] = c.x; ww[5] = c.y; ww[6] = c.z; ww[7] = c.w;
    } else {
        const uint4 a = p[0];
        ww[0] = a.x; ww[1] = a.y; ww[2] = a.z; ww[3] = a.w;
    }
}

// Prepares the wave's window (a word per lane; 2-bit: lanes 0-31) into its
// slice; the words of a unit are consecutive lanes, so the unit sums meet by
// butterfly. The slice is the wave's own: its LDS writes are ordered before
// its later reads without a workgroup barrier. PB: the pair layout of the
// weights (3 for 3-bit codes in the 4-bit geometry).
template <int BITS, bool BF16, int PB = BITS>
__device__ __forceinline__ void diag_prep_store(DiagSlice<BITS> &sl, const uint32_t (&ww)[16 / BITS], int lane) {
    using G = DiagGeom<BITS>;
    using P = Pairs<PB, BF16>;
    constexpr int VPW = 32 / BITS, WORDS = kDiagWindow / VPW, WPU = G::kUnitVals / VPW;
    float2 part = make_float2(0.f, 0.f);
    const int u = lane / WPU, wu = lane % WPU;
    if (lane < WORDS)
        prep_vals<BITS, BF16, PB>(ww, reinterpret_cast<uint32_t *>(sl.pairs + u * G::kStride) + wu * P::kCount, 1,
                              part);
#pragma unroll
    for (int m = 1; m < WPU; m <<= 1) {
        part.x += __shfl_xor(part.x, m, 64);
        part.y += __shfl_xor(part.y, m, 64);
    }
    if (lane < WORDS && wu == 0) sl.usum[u] = part;
    if (lane < 4 * G::kSteps) sl.zero[lane] = 0u;
}

// B operand of step t of the lane's unit (8 values: pairs 4 t .. 4 t + 3).
template <int BITS, bool BF16, int T>
__device__ __forceinline__ u32x4 diag_b(const u32x4 &unit, uint32_t magic_v) {
    using P = Pairs<BITS, BF16>;
    constexpr int word = (4 * T) / P::kCount, pb = (4 * T) % P::kCount;
    const uint32_t w = unit[word];
    return u32x4{expand_pair<BITS, BF16, pb>(w, magic_v), expand_pair<BITS, BF16, pb + 1>(w, magic_v),
                 expand_pair<BITS, BF16, pb + 2>(w, magic_v), expand_pair<BITS, BF16, pb + 3>(w, magic_v)};
}

// Sum over the 8 lanes sharing a row: the k-lanes (lanes 16 apart) and the
// two halves h of the row's line (lanes 8 apart). Every lane gets the same
// bits.
__device__ __forceinline__ float diag_row_sum(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(q[0]) + __uint_as_float(q[1]);
    // row_ror:8 -- lane n of each 16-lane row reads lane n +- 8
    const float o = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
    return (threadIdx.x & 8) ? o + v : v + o;
}

// s * (d - cx) + b * xs with 16-bit s, b.
template <bool BF16>
__device__ __forceinline__ float diag_fix(float d, uint16_t s, uint16_t b, float2 g) {
    return fmaf(to_float<BF16>(s), d - g.x, to_float<BF16>(b) * g.y);
}

// ---------------------------------------------------------------------------
// Router rows (ROUTER): the first sel.router_rows rows of the grid compute the
// logits instead of waiting for a logits kernel. Those rows are the shared
// expert's gate/up rows, which do their own work afterwards, then (if they are
// too few) rows of router work only; the routed rows come last. Workgroup b of
// the router rows takes experts b + n * w (n router workgroups, wave w <
// router_epw), one wave each, with the logits kernel's arithmetic
// (router_load_gate / router_pass: the same bits), and hands each token's
// logit to the routed rows as one tagged 64-bit word (poll_logits). The router
// rows wait for nothing and are dispatched first, so the routed rows that wait
// for them cannot hold them off the machine.
template <bool XBF16, int NCH>
__device__ __forceinline__ void router_row_expert(const RouterLaunch &L, int e, int lane, uint32_t tag) {
    u32x4 w[NCH];
    router_load_gate<NCH>(L, e, lane, w);
    for (int t = 0; t < L.tokens; ++t) {
        float acc[1];
        router_pass<XBF16, NCH, 1>(L, w, t, lane, acc);
        if (lane == 0) {
            const uint64_t v = (static_cast<uint64_t>(tag) << 32) | __float_as_uint(acc[0]);
            __hip_atomic_store(L.sync_logits + static_cast<int64_t>(t) * L.E + e, v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <bool XBF16>
__device__ __forceinline__ void router_rows_role(const RouterLaunch &L, int lane, int wave) {
    const int n = L.router_rows * static_cast<int>(gridDim.x);
    const int e = static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x) + n * wave;
    if (wave >= L.router_epw || e >= L.E) return;
    const uint32_t tag = sync_tag(__hip_atomic_load(L.sync_gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if (L.d == 1024) router_row_expert<XBF16, 2>(L, e, lane, tag);
    else if (L.d == 2048) router_row_expert<XBF16, 4>(L, e, lane, tag);
    else router_row_expert<XBF16, 8>(L, e, lane, tag);
}

// ---------------------------------------------------------------------------
// SELECT: the routes' slots are not chosen yet -- wave 0 of each routed
// workgroup runs the top-k selection of its token on `sel`'s logits (one
// partial row per token, E <= 256) while the other waves prepare x, and the
// workgroup (blockIdx.x 0, first route of the token) stores the token's
// choices for the down kernel and the caller. ROUTER (with SELECT): the
// logits come from the kernel's own router rows (above) instead.
template <int BITS, bool BF16, bool SELECT, bool ROUTER>
__global__ __launch_bounds__(64 * kDiagGateUpMaxWaves) void gateup_diag_kernel(
    RouteArgs ra, QProj gate, QProj up, QProj sgate, QProj sup, uint16_t *__restrict__ h,
    PrepVec hout, int down_bits, float limit, int fp32_swiglu, RouterLaunch sel) {
    // 3-bit codes run in the 4-bit geometry: each 16-byte unit of 4-bit
    // codes is a 12-byte piece of the 3-bit row, its words' values split
    // over their halves on arrival (the Pairs<3, *> layout)
    constexpr int CB = BITS == 3 ? 4 : BITS;
    using G = DiagGeom<CB>;
    constexpr int RT = kDiagGateUpTiles;
    constexpr int NI = 2 * G::kLines;   // loads per (tile, projection): row halves x lines
    __shared__ __align__(16) DiagSlice<CB> win[kDiagGateUpMaxWaves];
    __shared__ float red[kDiagGateUpMaxWaves][RT][2][16];
    __shared__ __align__(16) uint16_t hs[16 * RT];
    // scales and biases of the workgroup's rows: [gs, gb, us, ub][row][K / 64]
    // u16, rows padded by 16 bytes
    __shared__ __align__(16) uint8_t mlds[4 * 16 * RT * (2 * (4096 / 64) + 16)];
    // wave index in an SGPR: it feeds the loads' scalar offsets
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nl = lane & 15, kb = lane >> 4, hh = nl >> 3, r8 = nl & 7;
    static_assert(SELECT || !ROUTER, "router rows feed the in-kernel selection");
    int r = static_cast<int>(blockIdx.y);
    if constexpr (ROUTER) {
        // rows: [shared expert (router work first)] [router work only] [routed]
        const int y = r, S = sel.router_shared_rows;
        if (y < sel.router_rows) {
            router_rows_role<BF16>(sel, lane, wave);
            if (y >= S) return;
        }
        r = y < S ? ra.tokens * ra.top_k + y : y - sel.router_rows;
    }
    int token, slot;
    bool shared;
    if constexpr (SELECT) {
        const int routed = ra.tokens * ra.top_k;
        shared = r >= routed;
        token = shared ? r - routed : r / ra.top_k;
        slot = 0;
    } else {
        route_of(ra, r, token, slot, shared);
    }
    // the route's projections, field by field (selecting whole parameter
    // structs by reference would put them in scratch memory)
    const int N = gate.rows, K = gate.cols;
    const int n_slots = shared ? sgate.n_slots : gate.n_slots;
    const uint32_t *gwp = shared ? sgate.w : gate.w, *uwp = shared ? sup.w : up.w;
    const int64_t gw_slot = shared ? sgate.w_slot : gate.w_slot, uw_slot = shared ? sup.w_slot : up.w_slot;
    const int64_t gm_slot = shared ? sgate.m_slot : gate.m_slot, um_slot = shared ? sup.m_slot : up.m_slot;
    const int n0 = blockIdx.x * 16 * RT;
    const int wpr = K * BITS / 32, gpr = K / gate.group;
    const int waves = blockDim.x >> 6;   // = K / 512
    const int ug_log2 = units_per_group_log2<CB>(gate.group);
    DiagSlice<CB> &mw = win[wave];

    // Raw x of the window first (the prep waits only for it), then the
    // workgroup's scales and biases by whole lines, then the weights in
    // consumption order. The metadata geometry does not depend on the slot
    // and is worked out before any selection: thread i moves 16-byte pieces
    // i and i + 64 * waves of the four arrays' rows (meta_piece_of).
    uint32_t xw[16 / CB];
    diag_prep_load<CB>(xw, ra.x + static_cast<int64_t>(token) * K + wave * kDiagWindow, lane);
    const int mrs = 2 * gpr + 16;   // LDS bytes per metadata row
    // 4 arrays x 16 RT rows x gpr / 8 pieces: at most RT pieces per thread
    MetaPiece mp[RT];
#pragma unroll
    for (int q = 0; q < RT; ++q)
        mp[q] = meta_piece_of(static_cast<int>(threadIdx.x) + q * 64 * waves, 4, 16 * RT, gpr, mrs);
    if constexpr (SELECT) {
        __shared__ float2 stage[256];
        __shared__ int s_slot;
        if (!shared) {   // uniform across the workgroup
            // the sync generation first: polling compares against its tag
            uint32_t tag = 0;
            if constexpr (ROUTER)
                if (wave == 0)
                    tag = sync_tag(__hip_atomic_load(sel.sync_gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            // wave 1 also prepares wave 0's window while wave 0 selects
            uint32_t xw0[16 / CB];
            if (wave == 1) diag_prep_load<CB>(xw0, ra.x + static_cast<int64_t>(token) * K, lane);
            sched_fence();
            if (wave == 0) {
                // this route needs choice j only; the workgroup that stores the
                // token's choices (blockIdx.x 0, j 0) runs every round
                const int j = r - token * ra.top_k;
                const bool store = blockIdx.x == 0 && j == 0;
                const int rounds = store ? ra.top_k : j + 1;
                SelectOut o;
                if constexpr (ROUTER)
                    o = select_token_polled_any<4>(sel, token, tag, stage, rounds);
                else
                    o = select_token_any<1, 4>(sel, token, sel.logits + static_cast<int64_t>(token) * sel.E, 0, stage,
                                               rounds);
                const int sj = __builtin_amdgcn_readlane(o.slot, j);
                if (lane == 0) s_slot = sj;
                if (store) select_store(sel, token, o);
                if (waves == 1) diag_prep_store<CB, BF16, BITS>(mw, xw, lane);
            } else {
                diag_prep_store<CB, BF16, BITS>(mw, xw, lane);
                if (wave == 1) diag_prep_store<CB, BF16, BITS>(win[0], xw0, lane);
            }
            __syncthreads();
            slot = s_slot;
        } else {
            diag_prep_store<CB, BF16, BITS>(mw, xw, lane);
        }
    }
    sched_fence();
    const bool valid_slot = slot >= 0 && slot < n_slots;
    const int sl = valid_slot ? slot : 0;
    const int64_t mrow0 = static_cast<int64_t>(n0) * gpr;
    const uint16_t *m_gs = (shared ? sgate.s : gate.s) + sl * gm_slot + mrow0;
    const uint16_t *m_gb = (shared ? sgate.b : gate.b) + sl * gm_slot + mrow0;
    const uint16_t *m_us = (shared ? sup.s : up.s) + sl * um_slot + mrow0;
    const uint16_t *m_ub = (shared ? sup.b : up.b) + sl * um_slot + mrow0;
    u32x4 mv[RT];
#pragma unroll
    for (int q = 0; q < RT; ++q) {
        const uint16_t *arr = mp[q].arr == 0 ? m_gs : mp[q].arr == 1 ? m_gb : mp[q].arr == 2 ? m_us : m_ub;
        mv[q] = *reinterpret_cast<const u32x4 *>(arr + mp[q].off);
    }
    sched_fence();
    const uint32_t wbytes = 4u * 16 * RT * wpr;
    const int64_t wrow0 = static_cast<int64_t>(n0) * wpr;
    const __amdgpu_buffer_rsrc_t gw_rs = make_rsrc(gwp + sl * gw_slot + wrow0, wbytes);
    const __amdgpu_buffer_rsrc_t uw_rs = make_rsrc(uwp + sl * uw_slot + wrow0, wbytes);
    // load q = 2 * line + i: row 8 i + n % 8 of the tile, unit 4 h + kb of the line
    u32x4 wg[RT][NI], wu[RT][NI];
    // 3-bit codes: a window row is 192 bytes, twelve 16-byte pieces, and a
    // unit is 12 of them. Loads of single units would cover lines in part
    // (and be requested as partial lines); the wave reads its 16 RT window
    // rows whole instead, piece f = 64 j + lane of the rows' piece list in
    // load j (a tile's 16 rows are 3 loads), stages them in LDS one tile of
    // one projection at a time after the metadata barrier, and reads each
    // unit's three words back to split them.
    constexpr int P3 = kDiagWindow * 3 / 8 / 16;   // pieces per window row
    constexpr int NP3 = BITS == 3 ? 16 * RT * P3 / 64 : 1;
    static_assert(BITS != 3 || 16 * RT * P3 % 64 == 0, "whole loads per projection");
    u32x4 pg[NP3], pu[NP3];
    if constexpr (BITS == 3) {
#pragma unroll
        for (int j = 0; j < NP3; ++j) {
            const int f = 64 * j + lane, row = f / P3, pc = f - P3 * row;
            const uint32_t wo = 4u * static_cast<uint32_t>(row * wpr) + 16u * pc;
            pg[j] = __builtin_amdgcn_raw_buffer_load_b128(gw_rs, wo, 16 * P3 * wave, kAuxStream);
            pu[j] = __builtin_amdgcn_raw_buffer_load_b128(uw_rs, wo, 16 * P3 * wave, kAuxStream);
        }
    } else {
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
    }
    sched_fence();
    if constexpr (!SELECT) diag_prep_store<CB, BF16, BITS>(mw, xw, lane);
#pragma unroll
    for (int q = 0; q < RT; ++q)
        if (mp[q].store) *reinterpret_cast<u32x4 *>(mlds + mp[q].dst) = mv[q];
    __syncthreads();
    if constexpr (BITS == 3) {
        // the wave's own tile of rows in dynamic LDS (kDiag3RowWords words a
        // row, padded from 48 to spread the unit reads over the banks); each
        // tile's pieces overwrite the previous tile's after its reads
        extern __shared__ __align__(16) uint32_t stage3[];
        uint32_t *sw = stage3 + wave * (16 * kDiag3RowWords);
        constexpr int JT = NP3 / RT;   // loads per tile
        static_assert(16 * P3 == 64 * JT, "a tile's rows are whole loads");
        auto widen = [&](const u32x4(&pc)[NP3], u32x4(&out)[RT][NI]) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
                for (int jj = 0; jj < JT; ++jj) {
                    const int f = 64 * jj + lane, row = f / P3;
                    *reinterpret_cast<u32x4 *>(sw + kDiag3RowWords * row + 4 * (f - P3 * row)) = pc[JT * rt + jj];
                }
#pragma unroll
                for (int q = 0; q < NI; ++q) {
                    const int i = q & 1, line = q >> 1;
                    const uint32_t *u = sw + kDiag3RowWords * (8 * i + r8) + 3 * (8 * line + 4 * hh + kb);
                    out[rt][q] = spread3_halves(u[0], u[1], u[2]);
                }
            }
        };
        widen(pg, wg);
        widen(pu, wu);
    }
    const uint32_t magic_v = opaque_vgpr(Pairs<BITS, BF16>::kMagic);
    // diagonal A: lane (m, kb) feeds unit 8 line + 4 ((m / 2) % 2) + kb when m / 4 == kb
    const bool diag = (nl >> 2) == kb;
    const int ah = (nl >> 1) & 1;
    const int as = 16 * RT * mrs / 2;   // u16 between metadata arrays
    float accg[RT][2], accu[RT][2];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 2; ++i) accg[rt][i] = accu[rt][i] = 0.f;
#pragma unroll
    for (int line = 0; line < G::kLines; ++line) {
        const int uA = 8 * line + 4 * ah + kb;
        const uint8_t *abase =
            diag ? mw.pairs + uA * G::kStride : reinterpret_cast<const uint8_t *>(mw.zero);
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
        // the lane's unit 4 h + kb of this line, rows 8 i + n % 8 of each tile
        const int uB = 8 * line + 4 * hh + kb;
        const float2 us = mw.usum[uB];
        const int grp = (G::kUnits * wave + uB) >> ug_log2;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint16_t *m0 = reinterpret_cast<const uint16_t *>(mlds + (16 * rt + 8 * i + r8) * mrs) + grp;
                accg[rt][i] += diag_fix<BF16>(hh ? dg[rt][i][2] : dg[rt][i][0], m0[0], m0[as], us);
                accu[rt][i] += diag_fix<BF16>(hh ? du[rt][i][2] : du[rt][i][0], m0[2 * as], m0[3 * as], us);
            }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float g = diag_row_sum(accg[rt][i]);
            const float u = diag_row_sum(accu[rt][i]);
            if (lane < 8) {
                red[wave][rt][0][8 * i + lane] = g;
                red[wave][rt][1][8 * i + lane] = u;
            }
        }
    __syncthreads();
    if (wave != 0) return;
    // Wave 0: the 32 rows' h in window order, then h's prepared form (the
    // rows are whole words of the down input and one half of a 64-block).
    if (lane < 16 * RT) {
        const int rt = lane >> 4, n = lane & 15;
        float g = 0.f, u = 0.f;
        for (int w = 0; w < waves; ++w) {
            g += red[w][rt][0][n];
            u += red[w][rt][1][n];
        }
        uint16_t out = 0;
        if (valid_slot) out = swiglu16<BF16>(round16<BF16>(g), round16<BF16>(u), limit, fp32_swiglu != 0);
        h[static_cast<int64_t>(r) * N + n0 + lane] = out;
        hs[lane] = out;
    }
    const int vpw = 32 / down_bits, words = 16 * RT / vpw;
    if (lane < words) {
        const int unit = n0 / vpw + lane;
        prep_unit_at<BF16>(down_bits, &hs[lane * vpw],
                           hout.pairs + r * hout.pairs_stride + unit * pairs_per_word<BF16>(down_bits),
                           hout.parts + r * hout.parts_stride + unit);
    }
}

// Launch shape: one workgroup per (32 rows, route) with K / 512 waves, plus
// the rows of router work only when the kernel computes the logits itself.
template <int BITS, bool BF16>
hipError_t launch_gateup_diag(const DecodeLaunch &L, hipStream_t st) {
    const int waves = L.gate.cols / kDiagWindow;
    const int rr = L.sel ? L.sel->router_rows - L.sel->router_shared_rows : 0;
    // the down kernel reads its input prepared in the width it computes in
    const int down_bits = lane_bits(L.down.bits);
    const size_t lds = BITS == 3 ? waves * kDiag3WaveBytes : 0;
    dim3 grid(L.gate.rows / (16 * kDiagGateUpTiles), L.routes + rr);
    if (L.sel && L.sel->router_rows > 0)
        hipLaunchKernelGGL((gateup_diag_kernel<BITS, BF16, true, true>), grid, dim3(64 * waves), lds, st, L.ra,
                           L.gate, L.up, L.sgate, L.sup, L.h, L.hprep, down_bits, L.limit, L.fp32_swiglu, *L.sel);
    else if (L.sel)
        hipLaunchKernelGGL((gateup_diag_kernel<BITS, BF16, true, false>), grid, dim3(64 * waves), lds, st, L.ra,
                           L.gate, L.up, L.sgate, L.sup, L.h, L.hprep, down_bits, L.limit, L.fp32_swiglu, *L.sel);
    else
        hipLaunchKernelGGL((gateup_diag_kernel<BITS, BF16, false, false>), grid, dim3(64 * waves), lds, st, L.ra,
                           L.gate, L.up, L.sgate, L.sup, L.h, L.hprep, down_bits, L.limit, L.fp32_swiglu,
                           RouterLaunch{});
    return hipGetLastError();
}

}  // namespace locali
