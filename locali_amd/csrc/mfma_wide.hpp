// Grouped expert kernels on the matrix cores for tiles of up to 64 positions
// (prefill and batched decode; tiles of one or two positions take the
// small-tile kernels of mfma_small.hpp).
//
// A workgroup covers 128 output rows of one tile with eight compute waves and
// four loader waves:
//
//   compute wave w owns rows 16 w .. 16 w + 15. Per 64-value block it expands
//     its rows' codes once into the B operand of v_mfma_f32_16x16x32 (one
//     v_bitop3_b32 per pair, magic + q * 4^j, see mfma_grouped.hpp) and runs
//     the two MFMA steps of the block for every active 16-position block of
//     the tile, the A operand being the positions' prepared activations read
//     from LDS; each block's result is scaled by the row's group scale in
//     fp32, and every four blocks one more MFMA k-group against the positions'
//     fixup operands adds the blocks' b * sum x - s * magic * sum x' (the
//     factorised affine GEMV of dsv4_kernels.py:75-79, see make_fix). Its
//     weight words arrive by one 16-byte
//     load per lane, chunk and projection, several chunks ahead in registers
//     (WideDepth); every load is issued unconditionally (past the end it
//     reads zero through an out-of-range offset), so the in-order
//     vector-memory counter lets a compute wave wait on nothing but its own
//     oldest weight chunk.
//   the loader waves stage the tile's prepared activations into LDS one stage
//     (two 64-value blocks, 256 bytes per position) at a time, sixteen
//     consecutive lanes reading one position's 256 bytes, several stages of
//     loads in flight per lane; the 16-byte parts are XOR-swizzled by
//     position so that the 16 positions an MFMA step reads hit distinct
//     banks. Two LDS stages alternate, one workgroup barrier per stage.
//     The positions' fixup operands travel with their stage (one 16-byte
//     load per position and block) into a ring of three stages.
//   before the loop every wave helps to stage the rows' scales and biases of
//     the whole K range with 16-byte loads (whole runs of a row), overlapped
//     with the first weight chunks and the positions' vectors.
//
// Each expert's weights are read once per tile of 64 positions; positions past
// the tile's count only cost their 16-position block's MFMA steps.
//
//   wide_gateup_kernel   h = swiglu(up, gate) rounded as the decode path; the
//                        epilogue prepares h for the down projection (the
//                        workgroup owns two whole 64-value blocks of h)
//   wide_down_kernel     y[pos] = round(down(h[pos]))
#pragma once

#include "mfma_grouped.hpp"

namespace locali {

constexpr int kWideTokens = 64;
constexpr int kWideBlocks = kWideTokens / 16;     // 16-position MFMA blocks per tile
constexpr int kWideRows = 128;                    // output rows per workgroup
constexpr int kWideCompute = kWideRows / 16;      // compute waves
constexpr int kWideLoaders = 4;
constexpr int kWideThreads = 64 * (kWideCompute + kWideLoaders);

// Loads in flight: weight chunks per compute wave (kRing) and activation
// stages per loader lane (kSets). Tiles with fewer active 16-position blocks
// spend less time per stage, so they look further ahead.
template <int NACT>
struct WideDepth {
    static constexpr int kRing = NACT <= 2 ? 8 : 4;
    static constexpr int kSets = NACT == 1 ? 8 : NACT == 2 ? 4 : NACT == 3 ? 3 : 2;
};
constexpr int kWideStageBytes = kWideTokens * 256;

// Dynamic LDS of a wide kernel with NPROJ projections over K columns (the
// kernels have no static LDS, so all of kWideMaxLds is theirs): two
// activation stages, then scales / biases [block][row][2 NPROJ] (16-bit) of
// the whole K range, then three stages of the positions' fixup operands
// [stage % 3][block of the stage][position], then the positions' vectors.
constexpr int kWideFixStages = 3;
__host__ __device__ constexpr size_t wide_meta_offset() { return 2 * kWideStageBytes; }
// Metadata rows per block in LDS: one spare row, so that the staging stores
// of lanes that hold different blocks of one row fall in different banks.
constexpr int kWideMetaRows = kWideRows + 1;
__host__ __device__ constexpr size_t wide_gs_offset(int K, int nproj) {
    return wide_meta_offset() + static_cast<size_t>(K / 64) * kWideMetaRows * 2 * nproj * sizeof(uint16_t);
}
__host__ __device__ constexpr size_t wide_tok_offset(int K, int nproj) {
    return wide_gs_offset(K, nproj) + kWideFixStages * 2 * kWideTokens * sizeof(uint4);
}
__host__ __device__ constexpr size_t wide_lds_bytes(int K, int nproj) {
    return wide_tok_offset(K, nproj) + kWideTokens * sizeof(int);
}
constexpr size_t kWideMaxLds = 160 * 1024;

template <int NPROJ>
struct WideLds {
    u32x4 (*a)[kWideTokens][16];   // [stage][position][swizzled 16-byte part]
    uint16_t *meta;
    u32x4 (*fix)[2][kWideTokens];  // [stage % 3][block of the stage][position]

    __device__ __forceinline__ WideLds(unsigned char *base, int K)
        : a(reinterpret_cast<u32x4(*)[kWideTokens][16]>(base)),
          meta(reinterpret_cast<uint16_t *>(base + wide_meta_offset())),
          fix(reinterpret_cast<u32x4(*)[2][kWideTokens]>(base + wide_gs_offset(K, NPROJ))) {}
};

// Scales and biases of the workgroup's rows for every block. Item (row r,
// 8-group piece c) is that piece of each of the 2 NPROJ arrays (arr[2 j] =
// scales, arr[2 j + 1] = biases of projection j, rows of the workgroup), one
// entry per 64-value block (bpg blocks per group). With P pieces per row
// dividing 64, a wave's 64 items are 64 / P rows x all P pieces of each
// (whole 128-byte lines per load instruction): lane l holds row l % (64 / P),
// piece l / (64 / P). One pass covers every item (kWideMetaMaxGroups groups
// per row at most, which the host checks), and loads go out for every thread
// (past the last item they repeat it), so that the waits that follow count
// loads exactly: the loop's first wait is for its first weight chunk, not
// for every chunk in flight.
constexpr int kWideMetaPass = 2;
constexpr int kWideMetaMaxGroups = kWideMetaPass * kWideThreads * 8 / kWideRows;
template <int NPROJ>
struct WideMetaStage {
    static constexpr int U = kWideMetaPass;
    uint4 v[U][2 * NPROJ];
    int items;

    // (row, piece) of item e, P = gpr / 8 pieces per row. When P divides 64 a
    // wave holds whole rows; otherwise lanes take consecutive rows of one
    // piece.
    __device__ __forceinline__ static void item(int e, int pieces, int &r, int &c) {
        if (64 % pieces == 0) {
            const int rpw = 64 / pieces, l = e & 63;
            r = (e >> 6) * rpw + l % rpw;
            c = l / rpw;
        } else {
            r = e % kWideRows;
            c = e / kWideRows;
        }
    }

    __device__ __forceinline__ void load(const uint16_t *const (&arr)[2 * NPROJ], int gpr, int base) {
#pragma unroll
        for (int it = 0; it < U; ++it) {
            const int e = min(base + it * kWideThreads + static_cast<int>(threadIdx.x), items - 1);
            int r, c;
            item(e, gpr / 8, r, c);
#pragma unroll
            for (int a = 0; a < 2 * NPROJ; ++a)
                v[it][a] = reinterpret_cast<const uint4 *>(arr[a] + static_cast<int64_t>(r) * gpr)[c];
        }
    }

    __device__ __forceinline__ void store(uint16_t *meta, int bpg, int base, int gpr) const {
#pragma unroll
        for (int it = 0; it < U; ++it) {
            const int e = base + it * kWideThreads + static_cast<int>(threadIdx.x);
            if (e >= items) break;
            int r, c;
            item(e, gpr / 8, r, c);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                uint32_t w[NPROJ];
#pragma unroll
                for (int j = 0; j < NPROJ; ++j)
                    w[j] = ((v[it][2 * j][q / 2] >> (16 * (q % 2))) & 0xffffu) |
                           (((v[it][2 * j + 1][q / 2] >> (16 * (q % 2))) & 0xffffu) << 16);
                for (int t = 0; t < bpg; ++t) {
                    uint16_t *dst = meta + (static_cast<int64_t>((c * 8 + q) * bpg + t) * kWideMetaRows + r) * (2 * NPROJ);
                    if constexpr (NPROJ == 2)
                        *reinterpret_cast<uint2 *>(dst) = make_uint2(w[0], w[1]);
                    else
                        *reinterpret_cast<uint32_t *>(dst) = w[0];
                }
            }
        }
    }
};

// Loader lane lt (0 .. 255): part lt % 16 of positions lt / 16 + 16 i,
// i < NACT (one 16-position block each), and the fixup operand of block
// lt % 2 of the stage of position min(lt / 2, 16 NACT - 1) (stored by lanes
// below 32 NACT). Every load is issued: a stage past the last reads zero
// through an out-of-range offset.
template <int NACT>
struct WideLoad {
    u32x4 a[NACT];
    u32x4 f;
};

template <int NACT>
struct WideLoader {
    __amdgpu_buffer_rsrc_t rs, frs;
    uint32_t off[NACT], foff;
    int part, p0, fp, fb;

    __device__ __forceinline__ void load(WideLoad<NACT> &r, int s, int nsteps) const {
        const uint32_t past = s < nsteps ? 0u : kPastEnd;
#pragma unroll
        for (int i = 0; i < NACT; ++i) r.a[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, off[i] | past, s * 256, 0);
        r.f = __builtin_amdgcn_raw_buffer_load_b128(frs, foff | past, s * 32, 0);
    }

    __device__ __forceinline__ void store(const WideLoad<NACT> &r, u32x4 (*st)[16], u32x4 (*fx)[kWideTokens],
                                          int lt) const {
#pragma unroll
        for (int i = 0; i < NACT; ++i) {
            const int pos = p0 + 16 * i;
            st[pos][part ^ (pos & 15)] = r.a[i];
        }
        if (lt < 32 * NACT) fx[fb][fp] = r.f;
    }
};

// The compute waves' B operand of one block: eight pairs per lane, two MFMA
// steps.
template <int BITS, bool BF16>
__device__ __forceinline__ void wide_b(const BlockW<MfmaGeom<BITS, BF16>::kWPL> &bw, uint32_t magic_v, u32x4 &b0,
                                       u32x4 &b1) {
    using G = MfmaGeom<BITS, BF16>;
    uint32_t e[8];
#pragma unroll
    for (int i = 0; i < G::kWPL; ++i)
        static_for<0, G::kNP>([&](auto pc) {
            constexpr int p = decltype(pc)::value;
            e[i * G::kNP + p] = expand_pair<BITS, BF16, p>(bw.w[i], magic_v);
        });
    b0 = u32x4{e[0], e[1], e[2], e[3]};
    b1 = u32x4{e[4], e[5], e[6], e[7]};
}

// Everything of a wide kernel up to the accumulators for a tile with NACT
// active 16-position blocks: staging, the loader waves' loop, the compute
// waves' loop. w[j]: projection j's weight words of the workgroup's rows;
// marr: their scales and biases (see WideMetaStage); vec(p) the
// prepared-input vector of position p < count. Returns with the compute
// waves' acc[j] filled and every wave past the last barrier. SB: bits of the
// stored codes (BITS, or 3 for 3-bit rows computed in the 4-bit geometry: a
// lane's 32 values of a chunk arrive as 12 bytes and are widened when the
// chunk is consumed).
template <int BITS, bool BF16, int NPROJ, int NACT, int SB, typename TokOf>
__device__ __forceinline__ void wide_body(mf32x4_t (&acc)[NPROJ][NACT], const WideLds<NPROJ> &L, const int32_t *tt,
                                          const uint32_t *const (&w)[NPROJ],
                                          const uint16_t *const (&marr)[2 * NPROJ], const MfmaVec &in, int n_vec,
                                          TokOf tokof, int K, int group, int count) {
    using G = MfmaGeom<BITS, BF16>;
    constexpr int WPL = G::kWPL, CB = G::kCB, SPC = CB / 2;
    const int nblk = K / 64, nsteps = nblk / 2, nchunks = nblk / CB;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, nl = lane & 15, kb = lane >> 4;
    static_assert(SB == BITS || (SB == 3 && BITS == 4), "3-bit codes run in the 4-bit geometry");
    const int wpr = K * SB / 32;
    const int gpr = K / group, bpg = group / 64;
#pragma unroll
    for (int j = 0; j < NPROJ; ++j)
#pragma unroll
        for (int tb = 0; tb < NACT; ++tb) acc[j][tb] = mf32x4_t{0.f, 0.f, 0.f, 0.f};

    // Prologue. What the loop's first step needs goes out first, since a
    // CU's loads leave in issue order at the rate the memory system drains
    // them: every wave's share of the scales and biases of the whole K range
    // and the compute waves' first two weight chunks, the loader waves' first
    // activation stage (addresses from the dispatch's token list, no
    // barrier); then the loaders' later stages; the compute waves' other
    // chunks only once stage 0 and the metadata are in LDS.
    WideMetaStage<NPROJ> ms;
    ms.items = kWideRows * (gpr / 8);   // at most U * kWideThreads: one pass
    auto stage_meta = [&]() { ms.store(L.meta, bpg, 0, gpr); };

    if (wave >= kWideCompute) {
        const int lt = threadIdx.x - 64 * kWideCompute;
        WideLoader<NACT> ld;
        ld.rs = make_rsrc(in.pairs, static_cast<uint32_t>(4 * in.pairs_stride * n_vec));
        ld.frs = make_rsrc(in.fix, static_cast<uint32_t>(sizeof(uint4) * in.fix_stride * n_vec));
        ld.part = lt & 15;
        ld.p0 = lt >> 4;
        ld.fp = min(lt >> 1, 16 * NACT - 1);
        ld.fb = lt & 1;
        // positions past the tile's count read token 0's vector (results
        // discarded); so does a lane that stores no fixup operand
#pragma unroll
        for (int i = 0; i < NACT; ++i) {
            const int p = ld.p0 + 16 * i;
            const int t = p < count ? tokof(p, tt) : 0;
            ld.off[i] = 4u * static_cast<uint32_t>(t * in.pairs_stride) + 16u * ld.part;
        }
        const int tf = lt < 32 * NACT && ld.fp < count ? tokof(ld.fp, tt) : 0;
        ld.foff = static_cast<uint32_t>(sizeof(uint4) * (tf * in.fix_stride + ld.fb));
        constexpr int SETS = WideDepth<NACT>::kSets;
        WideLoad<NACT> r[SETS];
        ld.load(r[0], 0, nsteps);
        ms.load(marr, gpr, 0);
#pragma unroll
        for (int q = 1; q < SETS; ++q) ld.load(r[q], q, nsteps);
        stage_meta();
        ld.store(r[0], L.a[0], L.fix[0], lt);
        __syncthreads();
        for (int s0 = 0; s0 < nsteps; s0 += SETS) {
#pragma unroll
            for (int q = 0; q < SETS; ++q) {
                const int s = s0 + q;
                ld.load(r[q], s + SETS, nsteps);   // r[q] held stage s, stored during step s - 1
                if (s < nsteps) {
                    if (s + 1 < nsteps) ld.store(r[(q + 1) % SETS], L.a[(s + 1) & 1], L.fix[(s + 1) % kWideFixStages], lt);
                    __syncthreads();
                }
            }
        }
        return;
    }
    // compute waves: rows 16 wave + nl of the workgroup
    const uint32_t wbytes = 4u * kWideRows * wpr;
    __amdgpu_buffer_rsrc_t wrs[NPROJ];
#pragma unroll
    for (int j = 0; j < NPROJ; ++j) wrs[j] = make_rsrc(w[j], wbytes);
    // a chunk of a row (128 or 256 values) is 64 bytes, 16 a lane; of 3-bit
    // codes 48 bytes, 12 a lane
    constexpr int kLaneBytes = SB == 3 ? 12 : 16;
    const uint32_t w_off = 4u * static_cast<uint32_t>((wave * 16 + nl) * wpr) + kLaneBytes * kb;
    constexpr int RING = WideDepth<NACT>::kRing;
    ChunkRaw<SB> ring[RING][NPROJ];
    auto load_w = [&](ChunkRaw<SB> (&dst)[NPROJ], int c) {
        const uint32_t past = c < nchunks ? 0u : kPastEnd;
#pragma unroll
        for (int j = 0; j < NPROJ; ++j) {
            if constexpr (SB == 3)
                dst[j] = __builtin_amdgcn_raw_buffer_load_b96(wrs[j], w_off | past, c * 48, kAuxStream);
            else
                dst[j] = __builtin_amdgcn_raw_buffer_load_b128(wrs[j], w_off | past, c * 64, kAuxStream);
        }
    };
    // the scales and biases first (staging waits for them), then two weight
    // chunks; the other chunks behind stage 0 and the metadata
    constexpr int FIRST = RING < 2 ? RING : 2;
    ms.load(marr, gpr, 0);
#pragma unroll
    for (int q = 0; q < FIRST; ++q) load_w(ring[q], q);
    const uint32_t magic_v = opaque_vgpr(G::P::kMagic);
    const int row = wave * 16 + nl;
    stage_meta();
    __syncthreads();   // stage 0 and the scales / biases
#pragma unroll
    for (int q = FIRST; q < RING; ++q) load_w(ring[q], q);
    for (int c0 = 0; c0 < nchunks; c0 += RING) {
#pragma unroll
        for (int q = 0; q < RING; ++q) {
            const int c = c0 + q;
            if (c < nchunks) {
                u32x4 wt[NPROJ];
#pragma unroll
                for (int j = 0; j < NPROJ; ++j) {
                    wt[j] = chunk_words<SB>(ring[q][j]);
                    transpose_words<WPL>(wt[j]);
                }
#pragma unroll
                for (int sp = 0; sp < SPC; ++sp) {
                    const int s = c * SPC + sp;
                    const u32x4(*st)[16] = L.a[s & 1];
#pragma unroll
                    for (int jb = 0; jb < 2; ++jb) {
                        const int blk = 2 * s + jb;
                        const uint16_t *mrow = L.meta + (static_cast<int64_t>(blk) * kWideMetaRows + row) * (2 * NPROJ);
                        uint32_t m[NPROJ];
                        if constexpr (NPROJ == 2) {
                            const uint2 mm = *reinterpret_cast<const uint2 *>(mrow);
                            m[0] = mm.x;
                            m[1] = mm.y;
                        } else {
                            m[0] = *reinterpret_cast<const uint32_t *>(mrow);
                        }
                        u32x4 a0[NACT], a1[NACT];
#pragma unroll
                        for (int tb = 0; tb < NACT; ++tb) {
                            const u32x4 *arow = st[16 * tb + nl];
                            a0[tb] = arow[(8 * jb + 2 * kb) ^ nl];
                            a1[tb] = arow[(8 * jb + 2 * kb + 1) ^ nl];
                        }
#pragma unroll
                        for (int j = 0; j < NPROJ; ++j) {
                            u32x4 b0, b1;
                            wide_b<BITS, BF16>(block_words<WPL>(wt[j], 2 * sp + jb), magic_v, b0, b1);
                            const float sc = to_float<BF16>(static_cast<uint16_t>(m[j]));
#pragma unroll
                            for (int tb = 0; tb < NACT; ++tb) {
                                mf32x4_t d = {0.f, 0.f, 0.f, 0.f};
                                d = mfma_16x16x32<BF16>(a0[tb], b0, d);
                                d = mfma_16x16x32<BF16>(a1[tb], b1, d);
#pragma unroll
                                for (int i = 0; i < 4; ++i) acc[j][tb][i] = fmaf(sc, d[i], acc[j][tb][i]);
                            }
                        }
                    }
                    if (s & 1) {
                        // affine terms of blocks 2s - 2 .. 2s + 1: k-lane kb takes block
                        // 2s - 2 + kb (stages s - 1 and s of the fixup ring)
                        const int blk = 2 * s - 2 + kb;
                        const u32x4(*fx)[kWideTokens] = L.fix[(kb < 2 ? s - 1 : s) % kWideFixStages];
                        const uint16_t *mrow = L.meta + (static_cast<int64_t>(blk) * kWideMetaRows + row) * (2 * NPROJ);
                        u32x4 fb[NPROJ];
                        if constexpr (NPROJ == 2) {
                            const uint2 mm = *reinterpret_cast<const uint2 *>(mrow);
                            fb[0] = fix_b(mm.x);
                            fb[1] = fix_b(mm.y);
                        } else {
                            fb[0] = fix_b(*reinterpret_cast<const uint32_t *>(mrow));
                        }
#pragma unroll
                        for (int tb = 0; tb < NACT; ++tb) {
                            const u32x4 fa = fx[kb & 1][16 * tb + nl];
#pragma unroll
                            for (int j = 0; j < NPROJ; ++j) acc[j][tb] = mfma_16x16x32<BF16>(fa, fb[j], acc[j][tb]);
                        }
                    }
                    __syncthreads();
                }
            }
            // the slot's words are consumed: refill it in place (no register
            // moves across iterations), unconditionally (exact load counts)
            load_w(ring[q], c + RING);
        }
    }
}

// Workgroup row y takes tile y. The dispatch lists the shared expert's tiles
// first: they hold every position (full 64-position tiles, the longest
// workgroups) and start with the launch instead of forming its tail. The
// record and the tile count are read together (the grid has one row per
// possible tile, so the record is in bounds), one dependent load fewer before
// the workgroup knows its tile.
__device__ __forceinline__ bool wide_tile(const TileArgs &ta, int n_slots, int &slot, int &first, int &count,
                                          bool &shared) {
    const int tile = static_cast<int>(blockIdx.y);
    const int4 rec = reinterpret_cast<const int4 *>(ta.tiles)[tile];
    const int nt = *ta.n_tiles;
    // the record and the count before the decision: neither load waits for the other
    asm volatile("" ::"s"(rec.x), "s"(rec.y), "s"(rec.z), "s"(nt));
    slot = rec.x;
    first = rec.y;
    count = rec.z;
    shared = slot == -2;
    return !(tile >= nt || count <= 0 || count > kWideTokens || count < ta.min_count ||
             (!shared && (slot < 0 || slot >= n_slots || first < 0 || first + count > ta.R)));
}

template <int BITS, bool BF16, int SB, int NACT>
__device__ __forceinline__ void wide_gateup_tile(const TileArgs &ta, const QProj &pg, const QProj &pu, int sl,
                                                 bool shared, int first, int count,
                                                 const MfmaVec &xin, const MfmaVec &hout, int down_bits, float limit,
                                                 int fp32_swiglu, unsigned char *wlds) {
    const int K = pg.cols;
    const WideLds<2> L(wlds, K);
    const int n0 = blockIdx.x * kWideRows;
    const int wpr = K * SB / 32, gpr = K / pg.group;
    const int64_t r0 = static_cast<int64_t>(n0) * gpr;
    const uint32_t *const w[2] = {pg.w + sl * pg.w_slot + static_cast<int64_t>(n0) * wpr,
                                  pu.w + sl * pu.w_slot + static_cast<int64_t>(n0) * wpr};
    const uint16_t *const marr[4] = {pg.s + sl * pg.m_slot + r0, pg.b + sl * pg.m_slot + r0,
                                     pu.s + sl * pu.m_slot + r0, pu.b + sl * pu.m_slot + r0};
    mf32x4_t acc[2][NACT];
    // position p's token: the shared expert's tiles hold tokens in order; a
    // routed tile's come from the dispatch's list
    wide_body<BITS, BF16, 2, NACT, SB>(acc, L, ta.tile_tok + static_cast<int64_t>(blockIdx.y) * kWideTokens, w, marr, xin,
                                   ta.n_vec, [&](int p, const int32_t *t) { return shared ? first + p - ta.R : t[p]; },
                                   K, pg.group, count);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nl = lane & 15, kb = lane >> 4;
    // h of the tile's positions x the workgroup's 128 rows, in LDS (stage 0's
    // activations are no longer read: every wave has passed the last barrier)
    uint16_t(*hs)[kWideRows] = reinterpret_cast<uint16_t(*)[kWideRows]>(&L.a[0][0][0]);
    if (wave < kWideCompute) {
#pragma unroll
        for (int tb = 0; tb < NACT; ++tb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int q = 16 * tb + 4 * kb + i;
                const uint16_t hv =
                    q < count ? swiglu16<BF16>(round16<BF16>(acc[0][tb][i]), round16<BF16>(acc[1][tb][i]), limit,
                                               fp32_swiglu != 0)
                              : static_cast<uint16_t>(0);
                hs[q][wave * 16 + nl] = hv;
                if (hout.plain && q < count)
                    hout.plain[(first + q) * 2 * hout.pairs_stride + n0 + wave * 16 + nl] = hv;
            }
        }
    }
    __syncthreads();
    // Prepared h for the down projection: rows [n0, n0 + 128) are whole words
    // and two whole 64-blocks of every position's h; the sums of a block's
    // words meet by butterfly over consecutive lanes.
    const int vpw_d = 32 / down_bits, wpw = kWideRows / vpw_d, wpb = 64 / vpw_d, w32 = 32 / vpw_d;
    const int n32 = pg.rows / 32;
    for (int u0 = 0; u0 < 16 * NACT * wpw; u0 += kWideThreads) {
        const int uu = u0 + static_cast<int>(threadIdx.x), q = uu / wpw, wd = uu % wpw;
        float2 part = make_float2(0.f, 0.f);
        const bool mine = q < count;
        if (mine)
            prep_unit_at<BF16>(down_bits, &hs[q][wd * vpw_d],
                               hout.pairs + (first + q) * hout.pairs_stride +
                                   (n0 / vpw_d + wd) * pairs_per_word<BF16>(down_bits),
                               &part);
        for (int m = 1; m < wpb; m <<= 1) {
            part.x += __shfl_xor(part.x, m, 64);
            part.y += __shfl_xor(part.y, m, 64);
            // the 32-value sums once the butterfly has met them (the small
            // down kernel's operands)
            if (2 * m == w32 && hout.sum32 && mine && wd % w32 == 0)
                hout.sum32[(first + q) * n32 + (n0 + wd * vpw_d) / 32] = part;
        }
        if (mine && wd % wpb == 0) hout.fix[(first + q) * hout.fix_stride + n0 / 64 + wd / wpb] = make_fix<BF16>(part);
    }
}

template <int BITS, bool BF16, int SB>
__global__ __launch_bounds__(kWideThreads) void wide_gateup_kernel(TileArgs ta, QProj gate, QProj up, QProj sgate,
                                                                   QProj sup, MfmaVec xin, MfmaVec hout,
                                                                   int down_bits, float limit, int fp32_swiglu) {
    extern __shared__ __align__(16) unsigned char wlds[];
    int slot, first, count;
    bool shared;
    if (!wide_tile(ta, gate.n_slots, slot, first, count, shared)) return;
    const QProj pg = shared ? sgate : gate;
    const QProj pu = shared ? sup : up;
    const int sl = shared ? 0 : slot;
    switch ((count + 15) >> 4) {
    case 1: wide_gateup_tile<BITS, BF16, SB, 1>(ta, pg, pu, sl, shared, first, count, xin, hout, down_bits, limit, fp32_swiglu, wlds); break;
    case 2: wide_gateup_tile<BITS, BF16, SB, 2>(ta, pg, pu, sl, shared, first, count, xin, hout, down_bits, limit, fp32_swiglu, wlds); break;
    case 3: wide_gateup_tile<BITS, BF16, SB, 3>(ta, pg, pu, sl, shared, first, count, xin, hout, down_bits, limit, fp32_swiglu, wlds); break;
    default: wide_gateup_tile<BITS, BF16, SB, 4>(ta, pg, pu, sl, shared, first, count, xin, hout, down_bits, limit, fp32_swiglu, wlds); break;
    }
}

template <int BITS, bool BF16, int SB, int NACT>
__device__ __forceinline__ void wide_down_tile(const TileArgs &ta, const QProj &p, int sl, int first, int count,
                                               const MfmaVec &hin, uint16_t *__restrict__ y, unsigned char *wlds) {
    const int N = p.rows, K = p.cols;
    const WideLds<1> L(wlds, K);
    const int n0 = blockIdx.x * kWideRows;
    const int wpr = K * SB / 32, gpr = K / p.group;
    const int64_t r0 = static_cast<int64_t>(n0) * gpr;
    const uint32_t *const w[1] = {p.w + sl * p.w_slot + static_cast<int64_t>(n0) * wpr};
    const uint16_t *const marr[2] = {p.s + sl * p.m_slot + r0, p.b + sl * p.m_slot + r0};
    mf32x4_t acc[1][NACT];
    wide_body<BITS, BF16, 1, NACT, SB>(acc, L, nullptr, w, marr, hin, ta.n_vec,
                                   [&](int q, const int32_t *) { return first + q; }, K, p.group, count);
    const int wave = threadIdx.x >> 6;
    if (wave >= kWideCompute) return;
    const int lane = threadIdx.x & 63, nl = lane & 15, kb = lane >> 4;
    const int n = n0 + wave * 16 + nl;
#pragma unroll
    for (int tb = 0; tb < NACT; ++tb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int q = 16 * tb + 4 * kb + i;
            if (q < count) y[static_cast<int64_t>(first + q) * N + n] = from_float<BF16>(acc[0][tb][i]);
        }
    }
}

template <int BITS, bool BF16, int SB>
__global__ __launch_bounds__(kWideThreads) void wide_down_kernel(TileArgs ta, QProj down, QProj sdown, MfmaVec hin,
                                                                 uint16_t *__restrict__ y) {
    extern __shared__ __align__(16) unsigned char wlds[];
    int slot, first, count;
    bool shared;
    if (!wide_tile(ta, down.n_slots, slot, first, count, shared)) return;
    const QProj p = shared ? sdown : down;
    const int sl = shared ? 0 : slot;
    switch ((count + 15) >> 4) {
    case 1: wide_down_tile<BITS, BF16, SB, 1>(ta, p, sl, first, count, hin, y, wlds); break;
    case 2: wide_down_tile<BITS, BF16, SB, 2>(ta, p, sl, first, count, hin, y, wlds); break;
    case 3: wide_down_tile<BITS, BF16, SB, 3>(ta, p, sl, first, count, hin, y, wlds); break;
    default: wide_down_tile<BITS, BF16, SB, 4>(ta, p, sl, first, count, hin, y, wlds); break;
    }
}

// SB: bits of the stored codes (3: 3-bit rows on the 4-bit kernels).
template <int BITS, bool BF16, int SB = BITS>
hipError_t launch_wide_stage(int which, const MfmaLaunch &L, hipStream_t st) {
    TileArgs ta = L.ta;
    if (which == 1) {
        ta.n_vec = L.tokens;
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&wide_gateup_kernel<BITS, BF16, SB>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kWideMaxLds));
        if (attr != hipSuccess) return attr;
        dim3 grid(L.gate.rows / kWideRows, L.max_tiles);
        // the epilogue prepares h in the geometry the down stage computes in
        hipLaunchKernelGGL((wide_gateup_kernel<BITS, BF16, SB>), grid, dim3(kWideThreads),
                           wide_lds_bytes(L.gate.cols, 2), st, ta, L.gate, L.up, L.sgate, L.sup, L.xin, L.hmid,
                           lane_bits(L.down.bits), L.limit, L.fp32_swiglu);
    } else {
        ta.n_vec = L.routes;
        ta.min_count = L.min_count_down;
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&wide_down_kernel<BITS, BF16, SB>),
            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kWideMaxLds));
        if (attr != hipSuccess) return attr;
        dim3 grid(L.down.rows / kWideRows, L.max_tiles);
        hipLaunchKernelGGL((wide_down_kernel<BITS, BF16, SB>), grid, dim3(kWideThreads), wide_lds_bytes(L.down.cols, 1),
                           st, ta, L.down, L.sdown, L.hmid, L.y);
    }
    return hipGetLastError();
}

}  // namespace locali
