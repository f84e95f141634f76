// Grouped expert kernels on the matrix cores (prefill, batched decode).
//
// A tile is (slot, first sorted position, up to 16 tokens) of the dispatch's
// slot-sorted route order. A workgroup of 4 waves covers 64 output rows of
// one tile; each wave owns 16 rows and computes the 16x16 (token x row) block
// with v_mfma_f32_16x16x32_{bf16,f16}:
//
//   B operand (weights): lane (row n = lane % 16, k-lane kb = lane / 16) owns
//     WPL whole 32-bit words of every 64-value block of row n and expands them
//     with one v_bitop3_b32 per pair into 16-bit floats magic + q * 4^j (fp16:
//     the magic removed exactly by one packed add) -- 8 values per MFMA step.
//     The words arrive by one 16-byte load per lane and projection (the four
//     k-lanes of a row read 64 contiguous bytes = 4 / WPL blocks) and are
//     transposed across the k-lanes with v_permlane16/32_swap so that each
//     lane again holds its WPL words of every block of the chunk.
//   A operand (activations): the same lane reads the matching prepared pairs
//     (x pre-scaled by 4^-j, see qgemv.hpp) of token m = lane % 16, so A and B
//     agree on every k slot whatever order the words put the codes in.
//   Per 64-value block the two MFMA steps start from zero and the affine
//     group terms are applied in fp32:  acc += s * (D - magic*sum x') + b * sum x
//     (the factorised affine GEMV of dsv4_kernels.py:75-79), with the per-block
//     sums of the tile's tokens staged in LDS.
//
//   mfma_prep_kernel     prepared pairs + per-64 sums of the tokens' x
//   mfma_gateup_kernel   h = swiglu(up, gate) rounded as the decode path; the
//                        epilogue prepares h for the down projection (the
//                        workgroup owns whole 64-value blocks of h)
//   mfma_down_kernel     y[pos] = round(down(h[pos]))
// Weights of a slot are streamed once per tile of 16 tokens; each wave keeps
// the next chunk (one 16-byte weight load per projection and the matching
// activations) in flight while it works on the current one.
#pragma once

#include "grouped_kernels.hpp"

namespace locali {

constexpr int kMfmaTileTokens = 16;
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

// One thread per (vector, word); the W64 words of a 64-block are consecutive
// lanes, so their sums meet by butterfly.
template <int BITS, bool BF16>
__global__ __launch_bounds__(256) void mfma_prep_kernel(const uint16_t *__restrict__ v, int n_vec, int K,
                                                        MfmaVec out) {
    using G = MfmaGeom<BITS, BF16>;
    const int words = K / G::kVPW;
    const int u = blockIdx.x * blockDim.x + threadIdx.x;
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
    if (vec < n_vec && w % G::kW64 == 0) out.gsum[vec * out.gsum_stride + w / G::kW64] = part;
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

__device__ __forceinline__ void load_block_a(u32x4 (&a)[2], __amdgpu_buffer_rsrc_t rsrc, uint32_t voff,
                                             int blk) {
    a[0] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, blk * 128, 0);
    a[1] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff + 16u, blk * 128, 0);
}

// Group scales and biases of the workgroup's 64 rows, staged once into LDS as
// meta[g][r] = {scale, bias} of each projection (16-bit each): in the loop a
// lane then reads its row's pair with one LDS load instead of issuing small
// global loads that the compiler would schedule next to their use. Staged
// with 16-byte global loads (8 groups of one row per array), all of a batch
// of two per thread issued before the first LDS store, so the prologue costs
// one memory round trip per batch (one batch up to K = 4096 at group 64).
template <int NPROJ>
__device__ __forceinline__ void stage_meta(uint16_t *meta, const uint16_t *const (&arr)[2 * NPROJ],
                                           int gpr, int bpg) {
    const int chunks = kMfmaRows * (gpr / 8);
    for (int e0 = threadIdx.x; e0 < chunks; e0 += 2 * blockDim.x) {
        uint4 v[2][2 * NPROJ];
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int e = e0 + it * blockDim.x;
            if (e < chunks) {
                const int r = e % kMfmaRows, c = e / kMfmaRows;
#pragma unroll
                for (int a = 0; a < 2 * NPROJ; ++a)
                    v[it][a] = reinterpret_cast<const uint4 *>(arr[a] + static_cast<int64_t>(r) * gpr)[c];
            }
        }
#pragma unroll
        for (int it = 0; it < 2; ++it) {
            const int e = e0 + it * blockDim.x;
            if (e >= chunks) break;
            const int r = e % kMfmaRows, c = e / kMfmaRows;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int g = c * 8 + q;
#pragma unroll
                for (int t = 0; t < 2; ++t) {   // one entry per 64-value block (bpg is 1 or 2)
                    if (t >= bpg) break;
                    uint16_t *dst = meta + (static_cast<int64_t>(g * bpg + t) * kMfmaRows + r) * (2 * NPROJ);
                    if constexpr (NPROJ == 2) {
                        uint2 pk;
                        pk.x = ((v[it][0][q / 2] >> (16 * (q % 2))) & 0xffffu) |
                               (((v[it][1][q / 2] >> (16 * (q % 2))) & 0xffffu) << 16);
                        pk.y = ((v[it][2][q / 2] >> (16 * (q % 2))) & 0xffffu) |
                               (((v[it][3][q / 2] >> (16 * (q % 2))) & 0xffffu) << 16);
                        *reinterpret_cast<uint2 *>(dst) = pk;
                    } else {
                        *reinterpret_cast<uint32_t *>(dst) = ((v[it][0][q / 2] >> (16 * (q % 2))) & 0xffffu) |
                                                             (((v[it][1][q / 2] >> (16 * (q % 2))) & 0xffffu) << 16);
                    }
                }
            }
        }
    }
}

// Two MFMA steps of one block for one projection, from zero.
template <int BITS, bool BF16>
__device__ __forceinline__ mf32x4_t block_mfma(const BlockW<MfmaGeom<BITS, BF16>::kWPL> &bw,
                                               const u32x4 (&a)[2], uint32_t magic_v) {
    using G = MfmaGeom<BITS, BF16>;
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < G::kWPL; ++i)
        static_for<0, G::kNP>([&](auto pc) {
            constexpr int p = decltype(pc)::value;
            e[i * G::kNP + p] = expand_pair<BITS, BF16, p>(bw.w[i], magic_v);
        });
    const u32x4 b0 = {e[0], e[1], e[2], e[3]}, b1 = {e[4], e[5], e[6], e[7]};
    mf32x4_t d = {0.f, 0.f, 0.f, 0.f};
    d = mfma_16x16x32<BF16>(a[0], b0, d);
    d = mfma_16x16x32<BF16>(a[1], b1, d);
    return d;
}

// Per-64 sums of the tile's 16 positions for every block, [blk][16] float2.
// The position of thread i is i % 16 for every entry it stages (blockDim is a
// multiple of 16), so its vector index is loaded once and every sum load is
// issued before the first LDS store.
__device__ __forceinline__ void stage_gsum(float2 *gsl, const MfmaVec &in, int nblk, int count,
                                           const TileArgs &ta, bool shared, int first, bool by_token) {
    const int q = threadIdx.x % kMfmaTileTokens;
    const int pos = first + min(q, count - 1);
    const int vec = by_token ? tile_token(ta, shared, pos) : pos;
    const float2 *src = in.gsum + vec * in.gsum_stride;
    const int per = nblk * kMfmaTileTokens;
    for (int e0 = threadIdx.x; e0 < per; e0 += 8 * blockDim.x) {
        float2 v[8];
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int e = e0 + it * blockDim.x;
            if (e < per) v[it] = src[e / kMfmaTileTokens];
        }
#pragma unroll
        for (int it = 0; it < 8; ++it) {
            const int e = e0 + it * blockDim.x;
            if (e < per) gsl[e] = v[it];
        }
    }
}

__device__ __forceinline__ void apply_block(mf32x4_t &acc, const mf32x4_t &d, float s, float b,
                                            const float2 *gsl_blk, int kb) {
    const float4 c01 = reinterpret_cast<const float4 *>(gsl_blk + 4 * kb)[0];
    const float4 c23 = reinterpret_cast<const float4 *>(gsl_blk + 4 * kb)[1];
    const float cx[4] = {c01.x, c01.z, c23.x, c23.z}, cy[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = fmaf(s, d[i] - cx[i], fmaf(b, cy[i], acc[i]));
}

template <int BITS, bool BF16>
__global__ __launch_bounds__(64 * kMfmaWaves) void mfma_gateup_kernel(
    TileArgs ta, QProj gate, QProj up, QProj sgate, QProj sup, MfmaVec xin, MfmaVec hout,
    int down_bits, float limit, int fp32_swiglu) {
    using G = MfmaGeom<BITS, BF16>;
    constexpr int WPL = G::kWPL;
    extern __shared__ __align__(16) float2 gsl[];                 // [nblk][16], then meta
    __shared__ __align__(16) uint16_t hs[kMfmaTileTokens][kMfmaRows];
    const int tile = blockIdx.y;
    if (tile >= *ta.n_tiles) return;
    const int slot = ta.tiles[4 * tile], first = ta.tiles[4 * tile + 1];
    const int count = ta.tiles[4 * tile + 2];
    const bool shared = slot == -2;
    const QProj &pg = shared ? sgate : gate;
    const QProj &pu = shared ? sup : up;
    if (count <= 0 || count > kMfmaTileTokens || count < ta.min_count ||
        (!shared && (slot < 0 || slot >= pg.n_slots || first < 0 || first + count > ta.R)))
        return;
    const int K = pg.cols, nblk = K / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nl = lane & 15, kb = lane >> 4;
    const int n0 = blockIdx.x * kMfmaRows;
    const int sl = shared ? 0 : slot;
    const int wpr = K / G::kVPW;
    const int gpr = K / pg.group, bpg = pg.group / 64;
    // x pairs of token m = nl; the workgroup's 64 rows of gate and up
    const int tok_a = tile_token(ta, shared, first + min(nl, count - 1));
    const __amdgpu_buffer_rsrc_t ra_rs = make_rsrc(xin.pairs, static_cast<uint32_t>(4 * xin.pairs_stride * ta.n_vec));
    const uint32_t a_off = 4u * static_cast<uint32_t>(tok_a * xin.pairs_stride + kb * WPL * G::kNP);
    const uint32_t wbytes = 4u * kMfmaRows * wpr;
    const __amdgpu_buffer_rsrc_t gw_rs = make_rsrc(pg.w + sl * pg.w_slot + static_cast<int64_t>(n0) * wpr, wbytes);
    const __amdgpu_buffer_rsrc_t uw_rs = make_rsrc(pu.w + sl * pu.w_slot + static_cast<int64_t>(n0) * wpr, wbytes);
    const uint32_t w_off = 4u * static_cast<uint32_t>((wave * 16 + nl) * wpr) + 16u * kb;
    // Two chunks alternate: the loads of chunk c + 1 are issued before the
    // math of chunk c, and scheduling barriers keep the compiler from sinking
    // them behind it. Chunk 0 is issued before the staging below.
    constexpr int CB = G::kCB;
    const int nchunks = nblk / CB;   // even
    u32x4 g0, u0, g1, u1;
    u32x4 a0[CB][2], a1[CB][2];
    auto load_chunk = [&](u32x4 &g, u32x4 &u, u32x4(&a)[CB][2], int c) {
        const uint32_t past = c < nchunks ? 0u : kPastEnd;
        g = __builtin_amdgcn_raw_buffer_load_b128(gw_rs, w_off | past, c * 64, kAuxStream);
        u = __builtin_amdgcn_raw_buffer_load_b128(uw_rs, w_off | past, c * 64, kAuxStream);
#pragma unroll
        for (int j = 0; j < CB; ++j) load_block_a(a[j], ra_rs, a_off | past, c * CB + j);
    };
    load_chunk(g0, u0, a0, 0);
    sched_fence();
    stage_gsum(gsl, xin, nblk, count, ta, shared, first, true);
    uint16_t *meta = reinterpret_cast<uint16_t *>(gsl + nblk * kMfmaTileTokens);   // [blk][64][4]
    {
        const int64_t r0 = static_cast<int64_t>(n0) * gpr;
        const uint16_t *const arr[4] = {pg.s + sl * pg.m_slot + r0, pg.b + sl * pg.m_slot + r0,
                                        pu.s + sl * pu.m_slot + r0, pu.b + sl * pu.m_slot + r0};
        stage_meta<2>(meta, arr, gpr, bpg);
    }
    const uint2 *lmeta = reinterpret_cast<const uint2 *>(meta) + wave * 16 + nl;   // + blk * 64
    __syncthreads();
    const uint32_t magic_v = opaque_vgpr(G::P::kMagic);
    mf32x4_t accg = {0.f, 0.f, 0.f, 0.f}, accu = {0.f, 0.f, 0.f, 0.f};
    auto math_chunk = [&](u32x4 g, u32x4 u, const u32x4(&a)[CB][2], int c) {
        transpose_words<WPL>(g);
        transpose_words<WPL>(u);
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int blk = c * CB + j;
            const uint2 m = lmeta[blk * kMfmaRows];
            const mf32x4_t dg = block_mfma<BITS, BF16>(block_words<WPL>(g, j), a[j], magic_v);
            const mf32x4_t du = block_mfma<BITS, BF16>(block_words<WPL>(u, j), a[j], magic_v);
            const float2 *gb_lds = gsl + blk * kMfmaTileTokens;
            apply_block(accg, dg, to_float<BF16>(static_cast<uint16_t>(m.x)),
                        to_float<BF16>(static_cast<uint16_t>(m.x >> 16)), gb_lds, kb);
            apply_block(accu, du, to_float<BF16>(static_cast<uint16_t>(m.y)),
                        to_float<BF16>(static_cast<uint16_t>(m.y >> 16)), gb_lds, kb);
        }
    };
    for (int c = 0; c < nchunks; c += 2) {
        load_chunk(g1, u1, a1, c + 1);
        sched_fence();
        math_chunk(g0, u0, a0, c);
        sched_fence();
        load_chunk(g0, u0, a0, c + 2);
        sched_fence();
        math_chunk(g1, u1, a1, c + 1);
        sched_fence();
    }
    // lane holds tokens q = 4 kb + i of row n
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = 4 * kb + i;
        hs[q][wave * 16 + nl] = q < count ? swiglu16<BF16>(round16<BF16>(accg[i]), round16<BF16>(accu[i]),
                                                           limit, fp32_swiglu != 0)
                                          : static_cast<uint16_t>(0);
    }
    __syncthreads();
    // Prepared h for the down projection: rows [n0, n0 + 64) are whole words
    // and one whole 64-block of every position's h.
    const int vpw_d = 32 / down_bits, wpw = kMfmaRows / vpw_d;
    const int u = threadIdx.x, q = u / wpw, wd = u % wpw;
    float2 part = make_float2(0.f, 0.f);
    const bool mine = u < kMfmaTileTokens * wpw && q < count;
    if (mine)
        prep_unit_at<BF16>(down_bits, &hs[q][wd * vpw_d],
                           hout.pairs + (first + q) * hout.pairs_stride +
                               (n0 / vpw_d + wd) * pairs_per_word<BF16>(down_bits),
                           &part);
    for (int m = 1; m < wpw; m <<= 1) {
        part.x += __shfl_xor(part.x, m, 64);
        part.y += __shfl_xor(part.y, m, 64);
    }
    if (mine && wd == 0) hout.gsum[(first + q) * hout.gsum_stride + n0 / 64] = part;
}

template <int BITS, bool BF16>
__global__ __launch_bounds__(64 * kMfmaWaves) void mfma_down_kernel(TileArgs ta, QProj down, QProj sdown,
                                                                    MfmaVec hin, uint16_t *__restrict__ y) {
    using G = MfmaGeom<BITS, BF16>;
    constexpr int WPL = G::kWPL;
    extern __shared__ __align__(16) float2 gsl[];
    const int tile = blockIdx.y;
    if (tile >= *ta.n_tiles) return;
    const int slot = ta.tiles[4 * tile], first = ta.tiles[4 * tile + 1];
    const int count = ta.tiles[4 * tile + 2];
    const bool shared = slot == -2;
    const QProj &p = shared ? sdown : down;
    if (count <= 0 || count > kMfmaTileTokens || count < ta.min_count ||
        (!shared && (slot < 0 || slot >= p.n_slots || first < 0 || first + count > ta.R)))
        return;
    const int N = p.rows, K = p.cols, nblk = K / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nl = lane & 15, kb = lane >> 4;
    const int n = blockIdx.x * kMfmaRows + wave * 16 + nl;
    const int sl = shared ? 0 : slot;
    const int wpr = K / G::kVPW;
    const int gpr = K / p.group, bpg = p.group / 64;
    const int n0 = blockIdx.x * kMfmaRows;
    const __amdgpu_buffer_rsrc_t ra_rs = make_rsrc(hin.pairs, static_cast<uint32_t>(4 * hin.pairs_stride * ta.n_vec));
    const uint32_t a_off =
        4u * static_cast<uint32_t>((first + min(nl, count - 1)) * hin.pairs_stride + kb * WPL * G::kNP);
    const __amdgpu_buffer_rsrc_t w_rs =
        make_rsrc(p.w + sl * p.w_slot + static_cast<int64_t>(n0) * wpr, 4u * kMfmaRows * wpr);
    const uint32_t w_off = 4u * static_cast<uint32_t>((wave * 16 + nl) * wpr) + 16u * kb;
    constexpr int CB = G::kCB;
    const int nchunks = nblk / CB;   // even
    u32x4 w0, w1;
    u32x4 a0[CB][2], a1[CB][2];
    auto load_chunk = [&](u32x4 &w, u32x4(&a)[CB][2], int c) {
        const uint32_t past = c < nchunks ? 0u : kPastEnd;
        w = __builtin_amdgcn_raw_buffer_load_b128(w_rs, w_off | past, c * 64, kAuxStream);
#pragma unroll
        for (int j = 0; j < CB; ++j) load_block_a(a[j], ra_rs, a_off | past, c * CB + j);
    };
    load_chunk(w0, a0, 0);
    sched_fence();
    stage_gsum(gsl, hin, nblk, count, ta, shared, first, false);
    uint16_t *meta = reinterpret_cast<uint16_t *>(gsl + nblk * kMfmaTileTokens);   // [blk][64][2]
    {
        const int64_t r0 = static_cast<int64_t>(n0) * gpr;
        const uint16_t *const arr[2] = {p.s + sl * p.m_slot + r0, p.b + sl * p.m_slot + r0};
        stage_meta<1>(meta, arr, gpr, bpg);
    }
    const uint32_t *lmeta = reinterpret_cast<const uint32_t *>(meta) + wave * 16 + nl;
    __syncthreads();
    const uint32_t magic_v = opaque_vgpr(G::P::kMagic);
    mf32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    auto math_chunk = [&](u32x4 w, const u32x4(&a)[CB][2], int c) {
        transpose_words<WPL>(w);
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const int blk = c * CB + j;
            const uint32_t m = lmeta[blk * kMfmaRows];
            const mf32x4_t d = block_mfma<BITS, BF16>(block_words<WPL>(w, j), a[j], magic_v);
            apply_block(acc, d, to_float<BF16>(static_cast<uint16_t>(m)),
                        to_float<BF16>(static_cast<uint16_t>(m >> 16)), gsl + blk * kMfmaTileTokens, kb);
        }
    };
    for (int c = 0; c < nchunks; c += 2) {
        load_chunk(w1, a1, c + 1);
        sched_fence();
        math_chunk(w0, a0, c);
        sched_fence();
        load_chunk(w0, a0, c + 2);
        sched_fence();
        math_chunk(w1, a1, c + 1);
        sched_fence();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = 4 * kb + i;
        if (q < count) y[static_cast<int64_t>(first + q) * N + n] = from_float<BF16>(acc[i]);
    }
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
};

template <int BITS, bool BF16>
hipError_t launch_mfma_stage(int which, const MfmaLaunch &L, hipStream_t st) {
    if (which == 0) {   // prepare x for gate/up
        const int words = L.gate.cols / MfmaGeom<BITS, BF16>::kVPW;
        const int64_t threads = static_cast<int64_t>(L.tokens) * words;
        hipLaunchKernelGGL((mfma_prep_kernel<BITS, BF16>), dim3((threads + 255) / 256), dim3(256), 0, st,
                           L.ta.x, L.tokens, L.gate.cols, L.xin);
    } else if (which == 1) {
        TileArgs ta = L.ta;
        ta.n_vec = L.tokens;
        const size_t lds = sizeof(float2) * (L.gate.cols / 64) * kMfmaTileTokens +
                           sizeof(uint16_t) * 4 * kMfmaRows * (L.gate.cols / 64);
        dim3 grid(L.gate.rows / kMfmaRows, L.max_tiles);
        hipLaunchKernelGGL((mfma_gateup_kernel<BITS, BF16>), grid, dim3(64 * kMfmaWaves), lds, st, ta,
                           L.gate, L.up, L.sgate, L.sup, L.xin, L.hmid, L.down.bits, L.limit,
                           L.fp32_swiglu);
    } else {
        TileArgs ta = L.ta;
        ta.n_vec = L.routes;
        const size_t lds = sizeof(float2) * (L.down.cols / 64) * kMfmaTileTokens +
                           sizeof(uint16_t) * 2 * kMfmaRows * (L.down.cols / 64);
        dim3 grid(L.down.rows / kMfmaRows, L.max_tiles);
        hipLaunchKernelGGL((mfma_down_kernel<BITS, BF16>), grid, dim3(64 * kMfmaWaves), lds, st, ta,
                           L.down, L.sdown, L.hmid, L.y);
    }
    return hipGetLastError();
}

}  // namespace locali
