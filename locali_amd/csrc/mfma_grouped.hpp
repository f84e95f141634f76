// Shared pieces of the grouped expert kernels on the matrix cores
// (mfma_wide.hpp: tiles of up to 64 positions; mfma_small.hpp: one or two).
//
// v_mfma_f32_16x16x32_{bf16,f16} with
//   B operand (weights): lane (row n = lane % 16, k-lane kb = lane / 16) owns
//     WPL whole 32-bit words of every 64-value block of row n and expands them
//     with one v_bitop3_b32 per pair into 16-bit floats magic + q * 4^j (fp16:
//     the magic removed exactly by one packed add) -- 8 values per MFMA step.
//     The words arrive by one 16-byte load per lane and projection (the four
//     k-lanes of a row read 64 contiguous bytes = 4 / WPL blocks) and are
//     transposed across the k-lanes with v_permlane16/32_swap so that each
//     lane again holds its WPL words of every block of the chunk.
//   A operand (activations): the same lane supplies the matching prepared
//     pairs (x pre-scaled by 4^-j, see qgemv.hpp) of position m = lane % 16, so
//     A and B agree on every k slot whatever order the words put the codes in.
//   The affine group terms of the factorised affine GEMV (dsv4_kernels.py:
//     75-79), acc = sum_g s_g * (D_g - magic*sum x') + b_g * sum x, are split:
//     the kernels scale each block's two MFMA steps by its scale in fp32 and
//     add sum_g (b_g * xs_g - s_g * corr_g) with one more MFMA k-group per
//     block from the fixup operands (make_fix, fix_b).
//
//   mfma_prep_kernel     prepared pairs + per-64 fixup operands of the tokens' x
#pragma once

#include "grouped_kernels.hpp"

namespace locali {

constexpr int kMfmaWaves = 4;
constexpr int kMfmaRows = 16 * kMfmaWaves;
constexpr int kMfmaColsAlign = 512;   // cols: a whole number of chunk pairs at 2 and 4 bits

typedef float mf32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 mbf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 mf16x8_t __attribute__((ext_vector_type(8)));

template <bool BF16>
__device__ __forceinline__ mf32x4_t mfma_16x16x32(u32x4 a, u32x4 b, mf32x4_t c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mbf16x8_t, a),
                                                        __builtin_bit_cast(mbf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mf16x8_t, a),
                                                       __builtin_bit_cast(mf16x8_t, b), c, 0, 0, 0);
}

template <int BITS, bool BF16>
struct MfmaGeom {
    using P = Pairs<BITS, BF16>;
    static constexpr int kNP = P::kCount;        // pairs per word
    static constexpr int kVPW = 32 / BITS;       // values per word
    static constexpr int kW64 = 64 / kVPW;       // words per 64-value block
    static constexpr int kWPL = kW64 / 4;        // words per lane per block
    static constexpr int kCB = 4 / kWPL;         // blocks per 16-byte load (a chunk)
    static_assert(kWPL * kNP == 8, "one block = two MFMA steps of 4 pairs per lane");
};

// Fixup operand of one 64-value block from its sums part = (corr, xs): each
// split into three 16-bit parts (hi + mid + lo hold about 24 significant
// bits, as fp32), [xs_hi, xs_mid, xs_lo, corr_hi, corr_mid, corr_lo, 0, 0].
// Against a row's fix_b operand [b, b, b, -s, -s, -s, 0, 0] one k-group of an
// MFMA adds b * xs - s * corr, the block's affine terms.
template <bool BF16>
__device__ __forceinline__ uint4 make_fix(float2 part) {
    uint16_t x[3], c[3];
    float vx = part.y, vc = part.x;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        x[i] = from_float<BF16>(vx);
        vx -= to_float<BF16>(x[i]);
        c[i] = from_float<BF16>(vc);
        vc -= to_float<BF16>(c[i]);
    }
    return make_uint4(x[0] | (static_cast<uint32_t>(x[1]) << 16), x[2] | (static_cast<uint32_t>(c[0]) << 16),
                      c[1] | (static_cast<uint32_t>(c[2]) << 16), 0u);
}

// The row's half of that product from its packed (scale | bias << 16).
__device__ __forceinline__ u32x4 fix_b(uint32_t sb) {
    const uint32_t sc = sb & 0xffffu, b = sb >> 16, ns = sc ^ 0x8000u;
    return u32x4{b | (b << 16), b | (ns << 16), ns | (ns << 16), 0u};
}

// One thread per (vector, word); the W64 words of a 64-block are consecutive
// lanes, so their sums meet by butterfly.
template <int BITS, bool BF16>
__device__ __forceinline__ void mfma_prep_block(const uint16_t *__restrict__ v, int n_vec, int K, const MfmaVec &out,
                                                int block) {
    using G = MfmaGeom<BITS, BF16>;
    const int words = K / G::kVPW;
    const int u = block * 256 + static_cast<int>(threadIdx.x);
    const int vec = u / words, w = u % words;
    float2 part = make_float2(0.f, 0.f);
    if (vec < n_vec)
        prep_word<BITS, BF16>(v + static_cast<int64_t>(vec) * K + w * G::kVPW,
                              out.pairs + vec * out.pairs_stride + w * G::kNP, 1, part);
#pragma unroll
    for (int m = 1; m < G::kW64; m <<= 1) {
        part.x += __shfl_xor(part.x, m, 64);
        part.y += __shfl_xor(part.y, m, 64);
    }
    if (vec < n_vec && w % G::kW64 == 0) out.fix[vec * out.fix_stride + w / G::kW64] = make_fix<BF16>(part);
}

template <int BITS, bool BF16>
__global__ __launch_bounds__(256) void mfma_prep_kernel(const uint16_t *__restrict__ v, int n_vec, int K,
                                                        MfmaVec out) {
    mfma_prep_block<BITS, BF16>(v, n_vec, K, out, static_cast<int>(blockIdx.x));
}

// The dispatch's placement step and the preparation of the tokens' x in one
// launch: neither depends on the other, and each alone leaves most of the
// GPU idle. Blocks [0, place_blocks) place, the rest prepare.
template <int BITS, bool BF16>
__global__ __launch_bounds__(256) void place_prep_kernel(PlaceArgs pa, int place_blocks, const uint16_t *__restrict__ v,
                                                         int n_vec, int K, MfmaVec out) {
    const int b = static_cast<int>(blockIdx.x);
    if (b < place_blocks)
        dispatch_place_block(pa, b);
    else
        mfma_prep_block<BITS, BF16>(v, n_vec, K, out, b - place_blocks);
}

// Buffer resources: one 128-bit descriptor per array, held in SGPRs, so a
// load is "descriptor + per-lane 32-bit offset + per-block scalar offset"
// with no 64-bit address arithmetic per load, and out-of-range offsets read
// zero instead of faulting. (Descriptor word 3 for GFX9-family parts.)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

constexpr int kAuxStream = 2;   // non-temporal: weights are read once

// The lane's words of one 64-value block of one projection.
template <int WPL>
struct BlockW {
    uint32_t w[WPL];
};

// A 16-byte load gives k-lane kb the words [4 kb, 4 kb + 4) of the row's 64
// bytes; after the transpose k-lane kb holds words [kb * WPL, (kb + 1) * WPL)
// of each of the 4 / WPL blocks, block j in x[j * WPL + i]. v_permlane32_swap
// exchanges k-lanes {2, 3} of its first operand with k-lanes {0, 1} of its
// second, v_permlane16_swap k-lanes {1, 3} of the first with {0, 2} of the
// second: for one word per block the 4 x 4 transpose is the 32-swap of the
// register pairs (0, 2), (1, 3) and then the 16-swap of (0, 1), (2, 3); for
// two words per block the 2 x 2 transpose of word pairs is the 16-swap of
// (0, 2), (1, 3) and then the 32-swap of the same pairs.
template <int WPL>
__device__ __forceinline__ void transpose_words(u32x4 &x) {
    if constexpr (WPL == 1) {
        const auto a = __builtin_amdgcn_permlane32_swap(x[0], x[2], false, false);
        const auto b = __builtin_amdgcn_permlane32_swap(x[1], x[3], false, false);
        const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
        const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
        x = u32x4{c[0], c[1], d[0], d[1]};
    } else {
        static_assert(WPL == 2, "2- and 4-bit words");
        const auto a = __builtin_amdgcn_permlane16_swap(x[0], x[2], false, false);
        const auto b = __builtin_amdgcn_permlane16_swap(x[1], x[3], false, false);
        const auto c = __builtin_amdgcn_permlane32_swap(a[0], a[1], false, false);
        const auto d = __builtin_amdgcn_permlane32_swap(b[0], b[1], false, false);
        x = u32x4{c[0], d[0], c[1], d[1]};
    }
}

// A lane's share of one chunk of a row as it arrives from memory: the 16
// bytes of the 2- and 4-bit layouts, or (SB = 3: 3-bit codes computed in the
// 4-bit geometry) the 12 bytes of the same 32 values, widened to the 4-bit
// words by chunk_words once they have landed.
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
template <int SB>
using ChunkRaw = typename std::conditional<SB == 3, u32x3, u32x4>::type;

template <int SB>
__device__ __forceinline__ u32x4 chunk_words(const ChunkRaw<SB> &r) {
    if constexpr (SB == 3)
        return spread3_chunk(r[0], r[1], r[2]);
    else
        return r;
}

template <int WPL>
__device__ __forceinline__ BlockW<WPL> block_words(const u32x4 &x, int j) {
    BlockW<WPL> o;
#pragma unroll
    for (int i = 0; i < WPL; ++i) o.w[i] = x[j * WPL + i];
    return o;
}

// Offsets at or above 2^31 are outside every buffer here: such a load reads
// zero without touching memory (the pipeline's loads past the last chunk).
constexpr uint32_t kPastEnd = 0x80000000u;

__device__ __forceinline__ void apply_block(mf32x4_t &acc, const mf32x4_t &d, float s, float b,
                                            const float2 *gsl_blk, int kb) {
    const float4 c01 = reinterpret_cast<const float4 *>(gsl_blk + 4 * kb)[0];
    const float4 c23 = reinterpret_cast<const float4 *>(gsl_blk + 4 * kb)[1];
    const float cx[4] = {c01.x, c01.z, c23.x, c23.z}, cy[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = fmaf(s, d[i] - cx[i], fmaf(b, cy[i], acc[i]));
}

struct MfmaLaunch {
    TileArgs ta;
    QProj gate, up, down, sgate, sup, sdown;
    MfmaVec xin, hmid;
    float2 *hsum32;               // small tiles: sums of h per 32 values [routes][d_ff / 32]
    uint16_t *y;
    float limit;
    int32_t fp32_swiglu;
    int32_t max_tiles;
    int32_t tokens, routes;
    int32_t min_count_down;       // the down stage's ta.min_count (its small tiles may take more positions)
    PlaceArgs place;              // the dispatch's placement step (launched with the preparation)
    int32_t small_down_positions; // positions of the down stage's small tiles: 2 or 4 (mfma_small.hpp)
};

// Prepared pairs and per-64 sums of the tokens' x for the gate/up stage.
template <int BITS, bool BF16>
hipError_t launch_mfma_prep(const MfmaLaunch &L, hipStream_t st) {
    const int words = L.gate.cols / MfmaGeom<BITS, BF16>::kVPW;
    const int64_t threads = static_cast<int64_t>(L.tokens) * words;
    hipLaunchKernelGGL((mfma_prep_kernel<BITS, BF16>), dim3((threads + 255) / 256), dim3(256), 0, st, L.ta.x,
                       L.tokens, L.gate.cols, L.xin);
    return hipGetLastError();
}

// The dispatch's placement step (L.place) fused with that preparation.
template <int BITS, bool BF16>
hipError_t launch_place_prep(const MfmaLaunch &L, hipStream_t st) {
    const int words = L.gate.cols / MfmaGeom<BITS, BF16>::kVPW;
    const int64_t threads = static_cast<int64_t>(L.tokens) * words;
    const int place_blocks = (L.place.n_slots + kPlaceSlotsPerBlock - 1) / kPlaceSlotsPerBlock;
    const int64_t blocks = place_blocks + (threads + 255) / 256;
    hipLaunchKernelGGL((place_prep_kernel<BITS, BF16>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       L.place, place_blocks, L.ta.x, L.tokens, L.gate.cols, L.xin);
    return hipGetLastError();
}

}  // namespace locali
