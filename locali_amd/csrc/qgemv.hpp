// Wave-level affine-quantised GEMV core shared by the expert kernels.
//
// Lane geometry for a projection with K inputs at BITS per code:
//   VPC = 128 / BITS values per 16-byte chunk, CPR = K / VPC chunks per row.
//   LPR = min(64, CPR) lanes cooperate on one row; RPL = 64 / LPR rows are
//   covered by one wave-wide 16-byte load; each lane streams CPL = CPR / LPR
//   chunks of its row (chunk = lane_in_row + LPR * i), so a load instruction
//   reads 1 KiB of contiguous weights when LPR = 64.
//
// The activation slice a lane needs never changes across rows. A workgroup
// prepares it once in LDS (prep_vector: pre-scaled 16-bit pairs in the order
// the weight pairs are expanded, plus per-word partial sums), then every
// wave copies its lanes' slice into registers (XVec) and streams rows.
// All of a wave's weight words and group metadata are requested before any
// arithmetic, so the memory round trips of its rows overlap.
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
    float4 raw[CPL][2];     // per-word (corr, xs) as loaded, before xvec_finish
};

// LDS image of one prepared vector, lane-minor so that lane reads are
// conflict-free: pairs[i][wd][p][lane], part[i][wd][lane] = (corr, xs).
template <int BITS, bool BF16, int CPL, int LPR>
struct XLds {
    using P = Pairs<BITS, BF16>;
    uint32_t pairs[CPL][4][P::kCount][LPR];
    float2 part[CPL][4][LPR];
};

// 16-bit value times 2^E, exact for the powers of two used here.
template <bool BF16, int E>
__device__ __forceinline__ uint16_t scale_pow2(uint16_t v) {
    if constexpr (E == 0) return v;
    else return from_float<BF16>(ldexpf(to_float<BF16>(v), E));
}

// Prepare one word's worth of activations (VPW values at `src`).
// Prepare one word's worth of activations (32 / BITS values, given as 16-bit
// pairs in ww) into its pairs and partial sums (corr, xs).
// PB: the pair layout the products read (BITS, or 3 for 3-bit codes split
// over the halves of 4-bit-sized words).
template <int BITS, bool BF16, int PB = BITS>
__device__ __forceinline__ void prep_vals(const uint32_t (&ww)[16 / BITS], uint32_t *pairs,
                                          int pair_stride, float2 &part) {
    using P = Pairs<PB, BF16>;
    constexpr int VPW = 32 / BITS;
    uint16_t vals[VPW];
#pragma unroll
    for (int q = 0; q < VPW / 2; ++q) {
        vals[2 * q] = static_cast<uint16_t>(ww[q]);
        vals[2 * q + 1] = static_cast<uint16_t>(ww[q] >> 16);
    }
    float xs = 0.f, corr = 0.f;
#pragma unroll
    for (int q = 0; q < VPW; ++q) xs += to_float<BF16>(vals[q]);
    static_for<0, P::kCount>([&](auto pc) {
        constexpr PairSpec ps = P::kSpec[decltype(pc)::value];
        const uint16_t lo = scale_pow2<BF16, ps.lo_xexp>(vals[ps.lo_val]);
        const uint16_t hi = scale_pow2<BF16, ps.hi_xexp>(vals[ps.hi_val]);
        pairs[decltype(pc)::value * pair_stride] =
            static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
        if constexpr (!P::kSubtract)
            corr += P::kMagicValue * (to_float<BF16>(lo) + to_float<BF16>(hi));
    });
    part = make_float2(corr, xs);
}

template <int BITS, bool BF16>
__device__ __forceinline__ void prep_word(const uint16_t *__restrict__ src, uint32_t *pairs,
                                          int pair_stride, float2 &part) {
    uint32_t ww[16 / BITS];
    if constexpr (BITS == 2) {
        const uint4 a = *reinterpret_cast<const uint4 *>(src);
        const uint4 c = *reinterpret_cast<const uint4 *>(src + 8);
        ww[0] = a.x; ww[1] = a.y; ww[2] = a.z; ww[3] = a.w;
        ww[4] = c.x; ww[5] = c.y; ww[6] = c.z; ww[7] = c.w;
    } else if constexpr (BITS == 4) {
        const uint4 a = *reinterpret_cast<const uint4 *>(src);
        ww[0] = a.x; ww[1] = a.y; ww[2] = a.z; ww[3] = a.w;
    } else {
        const uint2 a = *reinterpret_cast<const uint2 *>(src);
        ww[0] = a.x; ww[1] = a.y;
    }
    prep_vals<BITS, BF16>(ww, pairs, pair_stride, part);
}

// Cooperative prep of a K-vector into LDS by `nthreads` threads.
template <int BITS, bool BF16, int CPL, int LPR>
__device__ __forceinline__ void prep_vector(XLds<BITS, BF16, CPL, LPR> &lds,
                                            const uint16_t *__restrict__ v, int tid, int nthreads) {
    constexpr int VPC = 128 / BITS, VPW = 32 / BITS;
    constexpr int units = LPR * CPL * 4;
    for (int u = tid; u < units; u += nthreads) {
        const int lane = u % LPR, wd = (u / LPR) % 4, i = u / (LPR * 4);
        const int k0 = (lane + LPR * i) * VPC + wd * VPW;
        prep_word<BITS, BF16>(v + k0, &lds.pairs[i][wd][0][lane], LPR, lds.part[i][wd][lane]);
    }
}

template <int BITS, bool BF16, int CPL, int LPR, int GPC>
__device__ __forceinline__ void load_xvec_lds(XVec<BITS, BF16, CPL, GPC> &xv,
                                              const XLds<BITS, BF16, CPL, LPR> &lds,
                                              int lane_in_row) {
    using P = Pairs<BITS, BF16>;
    constexpr int WPG = 4 / GPC;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
#pragma unroll
        for (int gp = 0; gp < GPC; ++gp) {
            float c = 0.f, s = 0.f;
#pragma unroll
            for (int wd = gp * WPG; wd < (gp + 1) * WPG; ++wd) {
                const float2 pt = lds.part[i][wd][lane_in_row];
                c += pt.x;
                s += pt.y;
            }
            xv.corr[i][gp] = c;
            xv.xs[i][gp] = s;
        }
#pragma unroll
        for (int wd = 0; wd < 4; ++wd)
#pragma unroll
            for (int p = 0; p < P::kCount; ++p) xv.xp[i][wd][p] = lds.pairs[i][wd][p][lane_in_row];
    }
}

// ---------------------------------------------------------------------------
// Prepared vectors in global memory. A vector of K values for a projection
// of BITS-bit codes is stored chunk-major: for chunk c (K range
// [c*VPC, (c+1)*VPC)) and word wd < 4, pairs[(c*4 + wd)*kCount + p] and
// part[c*4 + wd] = (corr, xs) -- the same per-word content XLds holds, laid
// out so that a lane reads its chunk with 16-byte loads. Prepared once per
// vector (by the router, a prep kernel, or the producing kernel's epilogue).
// ---------------------------------------------------------------------------
template <bool BF16>
__device__ __forceinline__ int pairs_per_word(int bits) {
    return bits == 2 ? Pairs<2, BF16>::kCount : bits == 4 ? Pairs<4, BF16>::kCount
                                                          : Pairs<8, BF16>::kCount;
}

// Prepare one word (32 / bits values starting at src) into its pairs and
// partial sums (runtime bit width). Word `unit` of a vector starts at value
// unit * (32 / bits) and lands at pairs + unit * pairs_per_word, part + unit.
template <bool BF16>
__device__ __forceinline__ void prep_unit_at(int bits, const uint16_t *src,
                                             uint32_t *__restrict__ pairs, float2 *__restrict__ part) {
    switch (bits) {
    case 2: prep_word<2, BF16>(src, pairs, 1, *part); break;
    case 4: prep_word<4, BF16>(src, pairs, 1, *part); break;
    default: prep_word<8, BF16>(src, pairs, 1, *part); break;
    }
}

// u32 pairs and float2 parts per prepared vector of K values.
__host__ __device__ inline int64_t prep_pairs_count(int K, int bits, bool bf16) {
    const int per_word = bits == 2 ? 8 : bits == 4 ? 4 : (bf16 ? 4 : 2);
    return static_cast<int64_t>(K) * bits / 32 * per_word;
}
__host__ __device__ inline int64_t prep_parts_count(int K, int bits) {
    return static_cast<int64_t>(K) * bits / 32;
}

template <int BITS, bool BF16, int CPL, int LPR, int GPC>
__device__ __forceinline__ void load_xvec_global(XVec<BITS, BF16, CPL, GPC> &xv,
                                                 const uint32_t *__restrict__ pairs,
                                                 const float2 *__restrict__ part, int lane_in_row) {
    using P = Pairs<BITS, BF16>;
    constexpr int N32 = 4 * P::kCount;         // u32 per chunk
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = lane_in_row + LPR * i;
        const uint32_t *src = pairs + static_cast<int64_t>(c) * N32;
        uint32_t buf[N32];
        if constexpr (N32 % 4 == 0) {
#pragma unroll
            for (int q = 0; q < N32 / 4; ++q) {
                const uint4 u = reinterpret_cast<const uint4 *>(src)[q];
                buf[4 * q] = u.x; buf[4 * q + 1] = u.y; buf[4 * q + 2] = u.z; buf[4 * q + 3] = u.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < N32; ++q) buf[q] = src[q];
        }
#pragma unroll
        for (int wd = 0; wd < 4; ++wd)
#pragma unroll
            for (int p = 0; p < P::kCount; ++p) xv.xp[i][wd][p] = buf[wd * P::kCount + p];
        xv.raw[i][0] = reinterpret_cast<const float4 *>(part + static_cast<int64_t>(c) * 4)[0];
        xv.raw[i][1] = reinterpret_cast<const float4 *>(part + static_cast<int64_t>(c) * 4)[1];
    }
}

// Folds the per-word sums loaded by load_xvec_global into per-group-part
// sums. Kept separate so that a kernel can issue its weight loads before
// anything waits on the activation loads.
template <int BITS, bool BF16, int CPL, int GPC>
__device__ __forceinline__ void xvec_finish(XVec<BITS, BF16, CPL, GPC> &xv) {
    constexpr int WPG = 4 / GPC;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const float4 pa = xv.raw[i][0], pb = xv.raw[i][1];
        const float2 pw[4] = {make_float2(pa.x, pa.y), make_float2(pa.z, pa.w),
                              make_float2(pb.x, pb.y), make_float2(pb.z, pb.w)};
#pragma unroll
        for (int gp = 0; gp < GPC; ++gp) {
            float cs = 0.f, xs = 0.f;
#pragma unroll
            for (int wd = gp * WPG; wd < (gp + 1) * WPG; ++wd) {
                cs += pw[wd].x;
                xs += pw[wd].y;
            }
            xv.corr[i][gp] = cs;
            xv.xs[i][gp] = xs;
        }
    }
}

// One row's weights and group metadata for one lane.
template <int CPL, int GPC>
struct RowData {
    u32x4 c[CPL];
    uint16_t s[CPL][GPC];
    uint16_t b[CPL][GPC];
};

// Group metadata of one row for one lane (scale and bias per group part).
template <int BITS, int CPL, int LPR, int GPC>
__device__ __forceinline__ void load_row_meta(RowData<CPL, GPC> &rd,
                                              const uint16_t *__restrict__ srow,
                                              const uint16_t *__restrict__ brow, int group,
                                              int lane_in_row) {
    using G = Geom<BITS, CPL, LPR, GPC>;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int k0 = (lane_in_row + LPR * i) * G::kVPC;
#pragma unroll
        for (int gp = 0; gp < GPC; ++gp) {
            const int g = (k0 + gp * G::kWPG * G::kVPW) / group;
            rd.s[i][gp] = srow[g];
            rd.b[i][gp] = brow[g];
        }
    }
}

// Eight 3-bit codes (the low 24 bits of v, LSB first) moved to the eight
// nibbles of a 4-bit word: 12-bit halves to 16-bit halves, 6-bit quarters to
// bytes, then each byte's two codes to its nibbles.
__device__ __forceinline__ uint32_t spread3_word(uint32_t v) {
    v = (v & 0x00000FFFu) | ((v << 4) & 0x0FFF0000u);
    v = (v & 0x003F003Fu) | ((v << 2) & 0x3F003F00u);
    return (v & 0x07070707u) | ((v << 1) & 0x70707070u);
}

// A 32-value chunk of 3-bit codes with each word's eight values split over
// its halves (values 0-3 at bits 0-11, 4-7 at bits 16-27; bits 12-15 and
// 28-31 hold other values' bits), the layout Pairs<3, *> reads: one shift
// and one bit select a word.
__device__ __forceinline__ uint32_t spread3_half(uint32_t v) {
    return ((v << 4) & 0xFFFF0000u) | (v & 0x0000FFFFu);
}
__device__ __forceinline__ u32x4 spread3_halves(uint32_t w0, uint32_t w1, uint32_t w2) {
    return u32x4{spread3_half(w0), spread3_half(__builtin_amdgcn_alignbit(w1, w0, 24)),
                 spread3_half(__builtin_amdgcn_alignbit(w2, w1, 16)), spread3_half(w2 >> 8)};
}

// A 32-value chunk of 3-bit codes (three words of the row's little-endian
// bit stream) as the chunk of 4-bit codes the 4-bit dot products read.
__device__ __forceinline__ u32x4 spread3_chunk(uint32_t w0, uint32_t w1, uint32_t w2) {
    return u32x4{spread3_word(w0 & 0xFFFFFFu), spread3_word(__builtin_amdgcn_alignbit(w1, w0, 24)),
                 spread3_word(__builtin_amdgcn_alignbit(w2, w1, 16)), spread3_word(w2 >> 8)};
}

// Packed weights of one row for one lane: CPL 16-byte chunks, streamed once.
// SB = 3: the row holds 3-bit codes (chunk c of 32 values is words 3c..3c+2)
// and each chunk is widened to 4-bit codes on load, for kernels built with
// the 4-bit geometry.
template <int CPL, int LPR, int GPC, int SB = 4>
__device__ __forceinline__ void load_row_weights(RowData<CPL, GPC> &rd,
                                                 const uint32_t *__restrict__ wrow,
                                                 int lane_in_row) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = lane_in_row + LPR * i;
        if constexpr (SB == 3) {
            const uint32_t *p = wrow + 3 * c;
            rd.c[i] = spread3_chunk(__builtin_nontemporal_load(p), __builtin_nontemporal_load(p + 1),
                                    __builtin_nontemporal_load(p + 2));
        } else {
            rd.c[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wrow) + c);
        }
    }
}

template <int BITS, int CPL, int LPR, int GPC, int SB = BITS>
__device__ __forceinline__ void load_row(RowData<CPL, GPC> &rd, const uint32_t *__restrict__ wrow,
                                         const uint16_t *__restrict__ srow,
                                         const uint16_t *__restrict__ brow, int group,
                                         int lane_in_row) {
    load_row_weights<CPL, LPR, GPC, SB>(rd, wrow, lane_in_row);
    load_row_meta<BITS, CPL, LPR, GPC>(rd, srow, brow, group, lane_in_row);
}

// Partial (this lane's chunks) of sum_k x_k w[row, k].
template <int BITS, bool BF16, int CPL, int LPR, int GPC>
__device__ __forceinline__ float row_partial(const RowData<CPL, GPC> &rd,
                                             const XVec<BITS, BF16, CPL, GPC> &xv,
                                             uint32_t magic_v) {
    using G = Geom<BITS, CPL, LPR, GPC>;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const uint32_t words[4] = {rd.c[i][0], rd.c[i][1], rd.c[i][2], rd.c[i][3]};
#pragma unroll
        for (int gp = 0; gp < GPC; ++gp) {
            float d = 0.f;
#pragma unroll
            for (int wd = gp * G::kWPG; wd < (gp + 1) * G::kWPG; ++wd)
                d = word_dot<BITS, BF16>(words[wd], xv.xp[i][wd], d, magic_v);
            const float sc = to_float<BF16>(rd.s[i][gp]);
            const float bi = to_float<BF16>(rd.b[i][gp]);
            acc = fmaf(sc, d - xv.corr[i][gp], fmaf(bi, xv.xs[i][gp], acc));
        }
    }
    return acc;
}

}  // namespace locali
