// Wave-level affine-quantised GEMV core shared by the decode kernels.
//
// Lane geometry for a projection with K inputs at BITS per code:
//   VPC = 128 / BITS values per 16-byte chunk, CPR = K / VPC chunks per row.
//   LPR = min(64, CPR) lanes cooperate on one row; RPL = 64 / LPR rows are
//   covered by one wave-wide 16-byte load; each lane streams CPL = CPR / LPR
//   chunks of its row (chunk = lane_in_row + LPR * i), so a load instruction
//   reads 1 KiB of contiguous weights when LPR = 64.
// The activation slice a lane needs never changes across rows, so it is
// loaded once, pre-scaled and packed into registers (XVec).
#pragma once

#include "common.hpp"

namespace locali {

struct QProj {
    const uint32_t *w;       // [slots, rows, cols * bits / 32]
    const uint16_t *s;       // [slots, rows, cols / group]
    const uint16_t *b;       // [slots, rows, cols / group]
    int32_t rows, cols, bits, group, n_slots;
    int64_t w_slot;          // words per slot
    int64_t m_slot;          // metadata elements per slot
};

template <int BITS, int CPL, int LPR, int GPC>
struct Geom {
    static constexpr int kVPC = 128 / BITS;       // values per chunk
    static constexpr int kVPW = 32 / BITS;        // values per word
    static constexpr int kRPL = 64 / LPR;         // rows per wave load
    static constexpr int kWPG = 4 / GPC;          // words per group part
    static_assert(GPC == 1 || GPC == 2, "group parts per chunk");
};

// Packed, pre-scaled activation slice of one lane plus its group constants.
template <int BITS, bool BF16, int CPL, int GPC>
struct XVec {
    using P = Pairs<BITS, BF16>;
    uint32_t xp[CPL][4][P::kCount];
    float corr[CPL][GPC];   // magic * sum of pre-scaled values per group part
    float xs[CPL][GPC];     // plain sum of values per group part
};

template <bool BF16>
__device__ __forceinline__ uint16_t scale_pow2(uint16_t v, int e) {
    if (e == 0) return v;
    return from_float<BF16>(ldexpf(to_float<BF16>(v), e));
}

// Load the lane's slice of a 16-bit vector (K values) into an XVec.
template <int BITS, bool BF16, int CPL, int LPR, int GPC>
__device__ __forceinline__ void load_xvec(XVec<BITS, BF16, CPL, GPC> &xv,
                                          const uint16_t *__restrict__ v,
                                          int lane_in_row) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    using P = Pairs<BITS, BF16>;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int k0 = (lane_in_row + LPR * i) * G::kVPC;
#pragma unroll
        for (int gp = 0; gp < GPC; ++gp) { xv.corr[i][gp] = 0.f; xv.xs[i][gp] = 0.f; }
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            uint16_t vals[G::kVPW];
            const uint16_t *src = v + k0 + wd * G::kVPW;
            if constexpr (G::kVPW == 16) {
                const uint4 a = *reinterpret_cast<const uint4 *>(src);
                const uint4 c = *reinterpret_cast<const uint4 *>(src + 8);
                const uint32_t ww[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    vals[2 * q] = static_cast<uint16_t>(ww[q]);
                    vals[2 * q + 1] = static_cast<uint16_t>(ww[q] >> 16);
                }
            } else if constexpr (G::kVPW == 8) {
                const uint4 a = *reinterpret_cast<const uint4 *>(src);
                const uint32_t ww[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    vals[2 * q] = static_cast<uint16_t>(ww[q]);
                    vals[2 * q + 1] = static_cast<uint16_t>(ww[q] >> 16);
                }
            } else {
                const uint2 a = *reinterpret_cast<const uint2 *>(src);
                const uint32_t ww[2] = {a.x, a.y};
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    vals[2 * q] = static_cast<uint16_t>(ww[q]);
                    vals[2 * q + 1] = static_cast<uint16_t>(ww[q] >> 16);
                }
            }
            const int gp = wd / G::kWPG;
            float s = 0.f;
#pragma unroll
            for (int q = 0; q < G::kVPW; ++q) s += to_float<BF16>(vals[q]);
            xv.xs[i][gp] += s;
#pragma unroll
            for (int p = 0; p < P::kCount; ++p) {
                const PairSpec ps = P::kSpec[p];
                const uint16_t lo = scale_pow2<BF16>(vals[ps.lo_val], ps.lo_xexp);
                const uint16_t hi = scale_pow2<BF16>(vals[ps.hi_val], ps.hi_xexp);
                xv.xp[i][wd][p] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
                xv.corr[i][gp] += P::kMagicValue * (to_float<BF16>(lo) + to_float<BF16>(hi));
            }
        }
    }
}

// Weights of one row for one lane: CPL chunks of 16 bytes.
template <int CPL>
struct RowChunks {
    u32x4 c[CPL];
};

template <int BITS, int CPL, int LPR>
__device__ __forceinline__ void load_row(RowChunks<CPL> &rc, const uint32_t *__restrict__ wrow,
                                         int lane_in_row) {
#pragma unroll
    for (int i = 0; i < CPL; ++i)
        rc.c[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4 *>(wrow) + lane_in_row + LPR * i);
}

// Partial (this lane's chunks) of sum_k x_k w[row, k].
template <int BITS, bool BF16, int CPL, int LPR, int GPC>
__device__ __forceinline__ float row_partial(const RowChunks<CPL> &rc,
                                             const XVec<BITS, BF16, CPL, GPC> &xv,
                                             const uint16_t *__restrict__ srow,
                                             const uint16_t *__restrict__ brow,
                                             int group, int lane_in_row) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const uint32_t words[4] = {rc.c[i][0], rc.c[i][1], rc.c[i][2], rc.c[i][3]};
        const int k0 = (lane_in_row + LPR * i) * G::kVPC;
#pragma unroll
        for (int gp = 0; gp < GPC; ++gp) {
            float d = 0.f;
#pragma unroll
            for (int wd = gp * G::kWPG; wd < (gp + 1) * G::kWPG; ++wd)
                d = word_dot<BITS, BF16>(words[wd], xv.xp[i][wd], d);
            const int g = (k0 + gp * G::kWPG * G::kVPW) / group;
            const float sc = to_float<BF16>(srow[g]);
            const float bi = to_float<BF16>(brow[g]);
            acc = fmaf(sc, d - xv.corr[i][gp], fmaf(bi, xv.xs[i][gp], acc));
        }
    }
    return acc;
}

}  // namespace locali
