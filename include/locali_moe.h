/*
 * Streamed-MoE layer on MI355X (gfx950): C ABI of liblocali_amd.so.
 *
 * All pointers are device pointers unless stated otherwise; `stream` is a
 * hipStream_t passed as void* (NULL = the default stream). Every entry point
 * validates shapes on the host, launches asynchronously, never synchronises
 * and never allocates device memory; scratch memory comes from a caller-owned workspace
 * whose size locali_moe_workspace_bytes() reports and which must be
 * zero-filled once before first use (the library leaves its counters at zero
 * after every call). Return value: 0 on success, a negative LOCALI_E_* code
 * otherwise; locali_moe_last_error() describes the last failure on the
 * calling thread. Grouped calls (locali_moe_forward, locali_moe_expert_grouped)
 * of 256 tokens or more run their small-tile kernels on a second stream of
 * the library's beside `stream`, forked from and joined back into `stream`
 * by events, so the call stays ordered on `stream` and can be captured into
 * a graph; that stream and its four events are created once per host thread
 * and device, on the first such call made outside stream capture
 * (locali_moe_forward_noalloc never creates them and keeps one stream). A call with tokens == 0 is an empty batch: it returns 0
 * and touches nothing (the reference returns an empty output).
 *
 * What each entry point replaces in the reference (MLX) implementation:
 *   locali_moe_router          the gate call V4ArenaMoE.route -> MoEGate
 *                              (dsv4_arena.py:165-166), Locali's own sigmoid
 *                              router ArenaMoE.route (arena.py:501-506), and
 *                              the expert -> slot lookup of ArenaMoE._apply
 *                              (arena.py:558-567)
 *   locali_moe_dispatch        the stable slot sort / segment of the mixed
 *                              tier path (arena.py:641-659)
 *   locali_moe_expert_decode   V4ArenaMoE._gather over a [T, k] slot grid
 *                              (dsv4_arena.py:168-235: gather_qmm up/gate,
 *                              clamped SwiGLU, gather_qmm down) fused with the
 *                              weighted combine (arena.py:619-624) and the
 *                              caller's shared-expert add (dsv4_engine.py:259)
 *   locali_moe_expert_grouped  the same expert math with (token, k) entries
 *                              grouped by slot (arena.py:641-672), one pass of
 *                              each slot's weights per group, then combine
 *                              (also exported as locali_moe_expert_prefill)
 *   locali_moe_combine         sum_k y * w in the activation dtype
 *                              (arena.py:623-624) or fp32 (arena.py:661-672)
 *   locali_moe_arena_fill      the slot fill ArenaStore._read_into/_read_many
 *                              (arena.py:179-200), as a host->HBM copy
 *   locali_moe_arena_fill_batch the fills of several slots in one kernel that
 *                              reads pinned host memory (same source lines)
 *   locali_moe_forward         ArenaMoE.__call__ (arena.py:508-547) for an
 *                              all-resident arena, plus the shared expert
 */
#ifndef LOCALI_MOE_H
#define LOCALI_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    LOCALI_DT_F32 = 0,
    LOCALI_DT_F16 = 1,
    LOCALI_DT_BF16 = 2,
};

enum {
    LOCALI_SCORE_SQRTSOFTPLUS = 0,
    LOCALI_SCORE_SIGMOID = 1,
    LOCALI_SCORE_SOFTMAX = 2,
};

enum {
    LOCALI_COMBINE_ROUNDED = 0,   /* y*w rounded to the activation dtype */
    LOCALI_COMBINE_FP32 = 1,      /* y*w and the sum kept in fp32 */
};

enum {
    LOCALI_OK = 0,
    LOCALI_E_ARG = -1,            /* invalid argument / unsupported shape */
    LOCALI_E_WORKSPACE = -2,      /* workspace too small */
    LOCALI_E_HIP = -4,            /* HIP runtime error */
};

/* One projection arena: every slot holds one expert's affine-quantised
 * matrix in MLX layout (reference arena.py:150-160 per (tier, proj, kind)):
 *   weight  uint32   [n_slots, rows, cols * bits / 32]  (codes as one
 *           little-endian bit stream per row, least-significant bits first;
 *           3-bit codes cross word boundaries, 32 values per 3 words)
 *   scales  dtype    [n_slots, rows, cols / group_size]
 *   biases  dtype    [n_slots, rows, cols / group_size]
 * rows = outputs, cols = inputs; dtype = meta_dtype (F16 or BF16), which must
 * equal the activation dtype (the reference casts activations to fp16 for
 * fp16 metadata, dsv4_arena.py:172-173). */
typedef struct {
    const void *weight;
    const void *scales;
    const void *biases;
    int32_t bits;          /* 2, 3, 4 or 8 */
    int32_t group_size;    /* 32, 64 or 128 */
    int32_t rows;
    int32_t cols;
    int32_t meta_dtype;    /* LOCALI_DT_F16 or LOCALI_DT_BF16 */
    int32_t n_slots;
} locali_qproj;

/* gate/up: rows = d_ff, cols = d_model; down: rows = d_model, cols = d_ff. */
typedef struct {
    locali_qproj gate;
    locali_qproj up;
    locali_qproj down;
} locali_expert_arena;

/* Router description (the checkpoint gate's tensors,
 * tf:modeling_deepseek_v4.py:1028-1033, 1062). */
typedef struct {
    const void *weight;            /* [n_experts, d_model] */
    int32_t weight_dtype;          /* LOCALI_DT_* */
    int32_t n_experts;             /* <= 512 */
    int32_t top_k;                 /* 1..16 */
    int32_t score_func;            /* LOCALI_SCORE_* */
    int32_t norm_topk;             /* renormalise selected scores */
    float routed_scale;            /* routed_scaling_factor */
    const float *score_bias;       /* [n_experts] selection-only bias, or NULL */
    const int32_t *tid2eid;        /* [vocab, top_k] hash routing table, or NULL */
    int32_t vocab;
} locali_router;

/* Workspace bytes for up to `tokens` tokens. */
size_t locali_moe_workspace_bytes(int32_t tokens, int32_t d_model, int32_t d_ff,
                                  int32_t n_experts, int32_t top_k,
                                  int32_t has_shared);

/* Router: idx/weights [tokens, top_k] (int32 / fp32); route_slot (optional,
 * int32 [tokens, top_k]) = slot_of_expert[idx] or -1. input_ids (int32
 * [tokens]) is used only with a hash table. logits_in (optional fp32
 * [tokens, n_experts]) skips the gate product. */
int locali_moe_router(const locali_router *router, const void *x, int32_t x_dtype,
                      int32_t tokens, int32_t d_model, const int32_t *input_ids,
                      const float *logits_in, const int32_t *slot_of_expert,
                      int32_t n_slots, int32_t *idx, float *weights,
                      int32_t *route_slot, void *workspace, size_t workspace_bytes,
                      void *stream);

/* Stable sort of the tokens*top_k route entries by slot. sorted_route
 * [tokens*top_k] holds route ids (t*top_k + j) grouped by ascending slot and
 * token order inside a slot; seg_start [n_slots + 1] is the exclusive prefix
 * count per slot. */
int locali_moe_dispatch(const int32_t *route_slot, int32_t tokens, int32_t top_k,
                        int32_t n_slots, int32_t *sorted_route, int32_t *seg_start,
                        void *stream);

/* Expert math over a [tokens, top_k] slot grid (+ one shared-expert route per
 * token when `shared` is non-NULL, read from its slot 0), fused with the
 * combine: out [tokens, d_model] in x_dtype. hidden: caller buffer of
 * (tokens*top_k + tokens) * d_ff 16-bit elements (post-SwiGLU activations).
 * Slots outside [0, n_slots) contribute zero. */
int locali_moe_expert_decode(const locali_expert_arena *routed,
                             const locali_expert_arena *shared, const void *x,
                             int32_t x_dtype, int32_t tokens, int32_t top_k,
                             const int32_t *route_slot, const float *weights,
                             float swiglu_limit, int32_t fp32_swiglu,
                             int32_t combine_mode, void *hidden, void *out,
                             void *workspace, size_t workspace_bytes, void *stream);

/* The two stages of locali_moe_expert_decode, callable separately:
 * gate/up + clamped SwiGLU into `hidden`, then down projection + combine
 * (+ shared) into `out`. The down stage reads the prepared hidden vectors the
 * gate/up stage leaves in the workspace, so both calls take the same
 * workspace. Same arguments and rules as expert_decode. */
int locali_moe_decode_gateup(const locali_expert_arena *routed,
                             const locali_expert_arena *shared, const void *x,
                             int32_t x_dtype, int32_t tokens, int32_t top_k,
                             const int32_t *route_slot, float swiglu_limit,
                             int32_t fp32_swiglu, void *hidden, void *workspace,
                             size_t workspace_bytes, void *stream);
int locali_moe_decode_down_combine(const locali_expert_arena *routed,
                                   const locali_expert_arena *shared,
                                   int32_t x_dtype, int32_t tokens, int32_t top_k,
                                   const int32_t *route_slot, const float *weights,
                                   int32_t combine_mode, void *out, void *workspace,
                                   size_t workspace_bytes, void *stream);

/* The decode forward's own first two kernels, callable separately (for a
 * caller that times or interleaves them; locali_moe_forward runs the same
 * kernels back to back):
 *   locali_moe_router_logits       logits [tokens, n_experts] fp32 = x . Wg^T
 *                                  (the gate product of V4ArenaMoE.route,
 *                                  dsv4_arena.py:165-166), tokens <= 8;
 *   locali_moe_decode_gateup_select gate/up + clamped SwiGLU with each token's
 *                                  routes chosen inside the kernel from those
 *                                  logits (score function, selection-only bias,
 *                                  top-k, renormalised and scaled weights, slot
 *                                  lookup: the rest of the gate and the
 *                                  expert -> slot lookup of arena.py:558-567),
 *                                  writing idx, weights, route_slot [tokens,
 *                                  top_k] and hidden; tokens <= 2, n_experts
 *                                  <= 256, gate/up of 2-, 3- or 4-bit codes
 *                                  in groups of 64 or 128, d_model a multiple
 *                                  of 512 up to 4096, d_ff a multiple of 32
 *                                  and a down projection of 2, 3 or 4 bits;
 *                                  the workspace is laid out as for
 *                                  locali_moe_decode_gateup, and
 *                                  locali_moe_decode_down_combine on the same
 *                                  workspace then finishes the layer. */
int locali_moe_router_logits(const locali_router *router, const void *x, int32_t x_dtype,
                             int32_t tokens, int32_t d_model, float *logits, void *stream);
int locali_moe_decode_gateup_select(const locali_router *router,
                                    const locali_expert_arena *routed,
                                    const locali_expert_arena *shared,
                                    const int32_t *slot_of_expert, const void *x,
                                    int32_t x_dtype, int32_t tokens, const int32_t *input_ids,
                                    const float *logits, float swiglu_limit,
                                    int32_t fp32_swiglu, int32_t *idx, float *weights,
                                    int32_t *route_slot, void *hidden, void *workspace,
                                    size_t workspace_bytes, void *stream);

/* Grouped form of locali_moe_expert_decode for many tokens: (token, k) entries
 * are grouped by slot on the device and every slot's weights are streamed
 * once per group; expert ids idx [tokens, top_k] and slot_of_expert [n_experts]
 * give the slots. Scratch comes from the workspace. */
int locali_moe_expert_grouped(const locali_expert_arena *routed,
                              const locali_expert_arena *shared, const void *x,
                              int32_t x_dtype, int32_t tokens, int32_t top_k,
                              int32_t n_experts, const int32_t *idx,
                              const int32_t *slot_of_expert, const float *weights,
                              float swiglu_limit, int32_t fp32_swiglu,
                              int32_t combine_mode, void *out, void *workspace,
                              size_t workspace_bytes, void *stream);

/* No counterpart in the reference: locali_moe_expert_grouped that also hands
 * out its intermediates, for stage-wise parity tests of the grouped kernels.
 * Positions p are the grouped order (routed routes sorted by slot, then the
 * shared expert's route of each token at R + t, R = tokens * top_k):
 * h_out [routes, d_ff] holds the gate/up + SwiGLU output of every position,
 * y_out [routes, d_model] the down projection rounded to the activation
 * dtype, route_pos_out [R] the position of route t * top_k + j. out is the
 * combined output as locali_moe_expert_grouped writes it. */
int locali_moe_expert_grouped_stages(const locali_expert_arena *routed,
                                     const locali_expert_arena *shared, const void *x,
                                     int32_t x_dtype, int32_t tokens, int32_t top_k,
                                     int32_t n_experts, const int32_t *idx,
                                     const int32_t *slot_of_expert, const float *weights,
                                     float swiglu_limit, int32_t fp32_swiglu,
                                     int32_t combine_mode, void *out, void *h_out,
                                     void *y_out, int32_t *route_pos_out, void *workspace,
                                     size_t workspace_bytes, void *stream);

/* The prefill entry point (the many-token path of V4ArenaMoE._gather,
 * dsv4_arena.py:168-235, grouped by slot as arena.py:641-672): the same call
 * as locali_moe_expert_grouped, under the name the decode / prefill split of
 * the layer gives it. */
int locali_moe_expert_prefill(const locali_expert_arena *routed,
                              const locali_expert_arena *shared, const void *x,
                              int32_t x_dtype, int32_t tokens, int32_t top_k,
                              int32_t n_experts, const int32_t *idx,
                              const int32_t *slot_of_expert, const float *weights,
                              float swiglu_limit, int32_t fp32_swiglu,
                              int32_t combine_mode, void *out, void *workspace,
                              size_t workspace_bytes, void *stream);

/* out[t] = round(sum_j round(y[t,j] * round(w[t,j]))) (ROUNDED) or the fp32
 * form (FP32), plus round(out + shared_y[t]) when shared_y is non-NULL.
 * y [tokens, top_k, d], shared_y [tokens, d], out [tokens, d] in dtype. */
int locali_moe_combine(const void *y, const void *shared_y, const float *weights,
                       int32_t dtype, int32_t tokens, int32_t top_k, int32_t d,
                       int32_t combine_mode, void *out, void *stream);

/* The combine of route outputs that sit anywhere in y: route (t, j) reads
 * row route_pos[t * top_k + j] of y (no term when negative), terms summed in
 * j order, rounded as locali_moe_combine rounds them (weights rounded to
 * out_dtype; ROUNDED: each product rounded; FP32: products and sum in fp32),
 * plus round(out + shared_y[t]) when shared_y is non-NULL. y rows [*, d] in
 * y_dtype (F32, F16 or BF16); shared_y, out [tokens, d] in out_dtype.
 * Replaces the unsort + fp32 scatter-add of routes that span tiers
 * (arena.py:657-672; the caller orders each token's routes tier by tier) and
 * the reassembly of a decode token's split hit / miss routes
 * (arena.py:605-618). */
int locali_moe_combine_routes(const void *y, int32_t y_dtype, const int32_t *route_pos,
                              const void *shared_y, const float *weights, int32_t out_dtype,
                              int32_t tokens, int32_t top_k, int32_t d, int32_t combine_mode,
                              void *out, void *stream);

/* Asynchronous host -> device copy of `bytes` into an arena slot region
 * (src should be pinned host memory for a truly asynchronous copy). */
int locali_moe_arena_fill(void *dst, const void *src_host, size_t bytes, void *stream);

/* One piece of a batched fill: `bytes` from host memory at src_host to device
 * memory at dst. */
typedef struct {
    void *dst;
    const void *src_host;
    size_t bytes;
} locali_fill_piece;

/* The records of several slot fills at once (ArenaStore._fill of several
 * experts, arena.py:179-200): pieces whose source is pinned host memory
 * visible to the device and whose addresses and sizes are multiples of 16
 * bytes are copied by one kernel that reads the host memory over PCIe (64
 * pieces per launch); any other piece by an asynchronous copy. The piece
 * table is read before the call returns; the host memory must stay until the
 * stream has passed the copy. */
int locali_moe_arena_fill_batch(const locali_fill_piece *pieces, int32_t n, void *stream);

/* The fills of n whole experts into their slots (the host-memory fills of
 * ArenaStore.submit, arena.py:356-435): expert i's records lie back to back
 * in host memory at src_host[i] (record a is slot_bytes[a] bytes), and record
 * a lands at dst_base[a] + slots[i] * slot_bytes[a], array a being the
 * slot-major device array of (projection, weight/scales/biases) a. Every
 * array holds n_slots slots; a slot outside [0, n_slots) fails the call with
 * LOCALI_E_ARG before anything is queued. Same copy kernel and rules as
 * locali_moe_arena_fill_batch. */
int locali_moe_arena_fill_slots(void *const *dst_base, const size_t *slot_bytes, int32_t n_arrays,
                                int32_t n_slots, const int32_t *slots, const void *const *src_host,
                                int32_t n, void *stream);

/* Whole layer on an all-resident arena: router, dispatch (decode or grouped
 * by token count), experts, combine, shared expert. out [tokens, d_model]. */
int locali_moe_forward(const locali_router *router, const locali_expert_arena *routed,
                       const locali_expert_arena *shared, const int32_t *slot_of_expert,
                       const void *x, int32_t x_dtype, int32_t tokens,
                       const int32_t *input_ids, float swiglu_limit,
                       int32_t fp32_swiglu, void *out, int32_t *idx, float *weights,
                       void *workspace, size_t workspace_bytes, void *stream);

/* No counterpart in the reference. For callers that cannot allocate (code
 * under HIP graph capture, tight serving loops): locali_moe_forward without
 * the workspace arguments. Its scratch is a static device array of
 * LOCALI_NOALLOC_SCRATCH_BYTES per GPU inside the library (enough for 64
 * tokens of a d_model 4096, 256-expert, d_ff 2048 layer with a shared
 * expert), set up and cleared by the first call on each device and held
 * until the process ends; a call needing more returns LOCALI_E_WORKSPACE.
 * It calls no allocator. All calls on one GPU share that GPU's array, so
 * calls that overlap on one GPU race: serialise them. */
#define LOCALI_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int locali_moe_forward_noalloc(const locali_router *router, const locali_expert_arena *routed,
                               const locali_expert_arena *shared, const int32_t *slot_of_expert,
                               const void *x, int32_t x_dtype, int32_t tokens,
                               const int32_t *input_ids, float swiglu_limit,
                               int32_t fp32_swiglu, void *out, int32_t *idx, float *weights,
                               void *stream);

/* No counterpart in the reference: a measurement helper. Reads `bytes`
 * (a multiple of 16, 16-byte aligned) of device memory once with the expert
 * kernels' 16-byte non-temporal loads and computes nothing (sink: `blocks`
 * words the kernel practically never writes). Timed over the decode step's
 * byte counts in dependent launches, it is the streaming floor the decode
 * kernels are compared with. */
int locali_moe_stream_read(const void *src, size_t bytes, uint32_t *sink, int32_t blocks, void *stream);

const char *locali_moe_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
