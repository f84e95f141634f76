// Host-side launch descriptors shared between the C-ABI layer (api.cpp) and
// the kernel translation units. Plain structs of device pointers and sizes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qgemv.hpp"

namespace locali {

// Routes of the decode path: r in [0, tokens*top_k) is (token r / top_k,
// slot route_slot[r]); r in [tokens*top_k, +tokens) is the shared expert of
// token r - tokens*top_k (slot 0 of the shared arena).
struct RouteArgs {
    const uint16_t *x;          // [tokens, d_model]
    const int32_t *route_slot;  // [tokens * top_k]
    int32_t tokens, top_k, n_shared;
};

struct CombineArgs {
    const float *weights;       // [tokens, top_k] router weights (fp32)
    uint16_t *out;              // [tokens, d_model]
    int32_t mode;               // 0: products rounded (single tier), 1: fp32 products
    uint32_t *gen;              // non-null: the decode sync generation, advanced once per call
};

// A batch of prepared vectors (see qgemv.hpp): vector v's pairs start at
// pairs + v * pairs_stride and its partial sums at parts + v * parts_stride.
struct PrepVec {
    uint32_t *pairs;
    float2 *parts;
    int64_t pairs_stride, parts_stride;
};

// Prepared inputs of the matrix-core grouped kernels, one vector per token
// or position: pairs [words * P] u32 (P pairs per word, as the decode
// layout) and fix [K / 64] of 8 16-bit values per 64-value block, the block's
// sums corr = magic * (sum of pre-scaled values) and xs = (sum of values)
// each split into three 16-bit parts: [xs_hi, xs_mid, xs_lo, corr_hi,
// corr_mid, corr_lo, 0, 0] (make_fix).
struct MfmaVec {
    uint32_t *pairs;
    uint4 *fix;
    int64_t pairs_stride, fix_stride;
    // optional (the grouped gate/up kernels' h, for stage-wise tests): the
    // vectors' plain values, [vec][2 * pairs_stride]
    uint16_t *plain;
    // optional (the 64-position gate/up kernel's h, for the small-tile down
    // kernel): each 32 values' sums (corr, xs), [vec][2 * pairs_stride / 32]
    float2 *sum32;
};

struct RouterLaunch;

// ---- batched host -> HBM fills (fill.hip) ------------------------------------
constexpr int kFillMaxPieces = 64;
struct FillBatch {
    int32_t n;
    int32_t first_block[kFillMaxPieces];    // first workgroup of each piece
    int64_t units[kFillMaxPieces];          // 16-byte units of each piece
    const void *src[kFillMaxPieces];        // device-visible address of pinned host memory
    void *dst[kFillMaxPieces];
};
hipError_t launch_fill(const FillBatch &b, int blocks, hipStream_t st);
int fill_blocks(int64_t units);

// ---- decode path -----------------------------------------------------------
struct DecodeLaunch {
    RouteArgs ra;
    PrepVec hprep;              // prepared hidden vectors, one per route (down geometry)
    int32_t routes;             // tokens * top_k + n_shared * tokens
    bool bf16;
    QProj gate, up, down;       // routed arena
    QProj sgate, sup, sdown;    // shared expert (slot 0), or copies of routed
    uint16_t *h;                // [routes, d_ff]
    float limit;
    int32_t fp32_swiglu;
    CombineArgs ca;
    // non-null: the routes' slots and weights are not chosen yet; the gate/up
    // kernel selects for its token from these logits and writes idx, weights
    // and route_slot (ra.route_slot, ca.weights point at the latter two)
    const RouterLaunch *sel;
};

// Bit width the kernels compute in: 3-bit codes are widened to 4-bit on load
// (the 4-bit kernels with 3-bit row loads), every other width is its own.
__host__ __device__ inline int lane_bits(int bits) { return bits == 3 ? 4 : bits; }

hipError_t launch_gateup_decode(const DecodeLaunch &L, hipStream_t st);
hipError_t launch_down_combine_decode(const DecodeLaunch &L, hipStream_t st);
int chunks_per_row(const QProj &p);
int group_parts(const QProj &p);

// Matrix-core decode gate/up kernel (mfma_decode.hpp): one wave per
// 512-value window of K and 16-row tile, workgroups of 2 tiles and K / 512
// waves. It takes 2-, 3- or 4-bit codes (gate and up alike; 3-bit rows are
// widened to 4-bit codes as they arrive) with groups of 64 or 128 (a
// metadata row of whole 16-byte pieces), K a multiple of 512 and at most
// 4096, d_ff a multiple of 32, and a down projection of 2, 3 or 4 bits (its
// epilogue prepares whole words of the down input, the decode layout the
// down kernel reads). The shared expert has the routed experts' shapes and
// quantisation.
constexpr int kDiagWindow = 512;
constexpr int kDiagGateUpTiles = 2;
constexpr int kDiagGateUpMaxWaves = 8;

inline bool gateup_diag_eligible(const DecodeLaunch &L) {
    auto ok = [](const QProj &p) {
        return (p.bits == 2 || p.bits == 3 || p.bits == 4) && (p.group == 64 || p.group == 128) &&
               (p.cols / p.group) % 8 == 0 && p.cols % kDiagWindow == 0;
    };
    return ok(L.gate) && ok(L.up) && L.gate.bits == L.up.bits &&
           (L.down.bits == 2 || L.down.bits == 3 || L.down.bits == 4) &&
           L.gate.cols / kDiagWindow <= kDiagGateUpMaxWaves && L.gate.rows % (16 * kDiagGateUpTiles) == 0;
}
hipError_t decode_diag_b2(const DecodeLaunch &L, hipStream_t st);
hipError_t decode_diag_b3(const DecodeLaunch &L, hipStream_t st);
hipError_t decode_diag_b4(const DecodeLaunch &L, hipStream_t st);

// ---- router ------------------------------------------------------------------
struct RouterLaunch {
    const uint16_t *x;          // [tokens, d] activations (bf16/fp16 bits)
    bool x_bf16;
    const void *gate_w;         // [E, d]
    int32_t gate_dtype;         // 0 fp32, 1 fp16, 2 bf16
    const float *bias;          // [E] selection-only bias or null
    const int32_t *tid2eid;     // [vocab, top_k] hash table or null
    const int32_t *input_ids;   // [tokens] or null
    int32_t vocab;
    int32_t tokens, d, E, top_k;
    int32_t score_func;         // 0 sqrtsoftplus, 1 sigmoid, 2 softmax
    int32_t norm_topk;
    float routed_scale;
    const int32_t *slot_of_expert;  // [E] or null
    int32_t n_slots;
    int32_t *idx;               // [tokens, top_k]
    float *weights;             // [tokens, top_k]
    int32_t *route_slot;        // [tokens, top_k] or null
    float *logits;              // workspace [tokens, E]
    const float *logits_in;     // optional precomputed logits [tokens, E]
    // Router rows of the fused decode kernel (router_rows > 0): the logits
    // travel through sync_logits as (tag, fp32 bits) words, tag =
    // sync_tag(*sync_gen); the down kernel of the same call advances the
    // generation, so a later call never mistakes these words for its own.
    uint64_t *sync_logits;      // [tokens, E]
    uint32_t *sync_gen;
    // The first router_rows rows of the fused grid compute the logits: the
    // first router_shared_rows of them are the shared expert's gate/up rows
    // (which wait for nothing), the rest are rows of router work only.
    int32_t router_rows;
    int32_t router_shared_rows;
    int32_t router_epw;         // experts (one per wave) per router workgroup
};

// Tag of a sync generation: odd, so zero-filled memory never matches.
__host__ __device__ inline uint32_t sync_tag(uint32_t gen) { return 2u * gen + 1u; }

// logits_only: launch only the logits kernel of the decode (gemv) path and
// leave the selection to the caller's kernel (router_select_fusable).
hipError_t launch_router(const RouterLaunch &L, hipStream_t st, bool logits_only = false);

// The decode gate/up kernel can select for its own token when the logits come
// from the gemv path (few tokens, no precomputed logits) into one partial row
// per token, and E <= 256.
constexpr int kFusedSelectMaxTokens = 8;
inline bool router_select_fusable(const RouterLaunch &L) {
    return !L.logits_in && L.tokens <= kFusedSelectMaxTokens && L.E <= 256 && L.top_k <= 16;
}

// The decode gate/up kernel can also compute the logits itself (router rows
// of workgroups dispatched ahead of its gate/up rows), for at most
// kFusedRouterMaxTokens tokens, a gate of the activations' 16-bit dtype and
// d_model of 1024, 2048 or 4096 (the logits kernel's fast path, whose bits it
// reproduces).
constexpr int kFusedRouterMaxTokens = 2;
constexpr int kSyncMaxExperts = 256;
inline bool router_rows_fusable(const RouterLaunch &L) {
    const bool dot_ok = L.gate_dtype != 0 && ((L.gate_dtype == 2) == L.x_bf16);
    return router_select_fusable(L) && L.tokens <= kFusedRouterMaxTokens && L.E <= kSyncMaxExperts && dot_ok &&
           (L.d == 1024 || L.d == 2048 || L.d == 4096);
}

// ---- grouped (prefill) path --------------------------------------------------
struct GroupedLaunch {
    const uint16_t *x;          // [tokens, d]
    bool bf16;
    int32_t tokens, top_k, n_shared, E;
    const int32_t *idx;         // [tokens, top_k] expert ids
    const int32_t *slot_of_expert;  // [E]
    QProj gate, up, down, sgate, sup, sdown;
    float limit;
    int32_t fp32_swiglu;
    const float *weights;       // [tokens, top_k]
    int32_t combine_mode;
    uint16_t *out;              // [tokens, d]
    // workspace
    int32_t *seg_offset;        // [E + 2]   segment starts (+ shared), last = total
    int32_t *seg_slot;          // [E + 1]
    int32_t *sorted_route;      // [tokens * top_k + tokens]  route ids in segment order
    int32_t *route_pos;         // [tokens * top_k + tokens]  inverse
    int32_t *tiles;             // [max_tiles * 4] (segment, first, count, pad)
    int32_t *n_tiles;           // [1]
    uint16_t *h;                // [routes, d_ff] in sorted order
    uint16_t *y;                // [routes, d]    in sorted order
    int32_t max_tiles;
    int32_t tile_tokens;
};

hipError_t launch_grouped(const GroupedLaunch &L, hipStream_t st);
int grouped_max_tiles(int tokens, int top_k, int n_shared, int E, int tile_tokens);
struct MfmaLaunch;
hipError_t launch_mfma(int which, bool bf16, const MfmaLaunch &L, hipStream_t st);

}  // namespace locali
