/*
 * Planner extension of liblocali_amd.so, beside the reference ABI of
 * locali_core.h (which stays identical to native/locali_core.h).
 *
 * locali_cache_plan_each plans `keys` in order like locali_cache_plan, except
 * that each key also sees as pinned every slot the keys before it in the same
 * call resolved to (a hit or a placement). It equals one locali_cache_plan
 * call per key with the pins growing by each result, which is how this
 * library's V4ArenaStore places a layer's experts (one expert per slot even
 * in a nearly full tier; the reference's single multi-key call,
 * dsv4_arena.py:86-90, can hand an earlier key's slot to a later miss) -- in
 * one call instead of one per key. Return codes and the state after a -3 as
 * locali_cache_plan.
 */
#ifndef LOCALI_PLANNER_H
#define LOCALI_PLANNER_H

#include "locali_core.h"

#ifdef __cplusplus
extern "C" {
#endif

int locali_cache_plan_each(locali_cache *cache, const int32_t *keys, size_t key_count,
                           const int32_t *pinned_slots, size_t pinned_count, int touch_hits,
                           locali_cache_result *results);

/*
 * Device-resident planner. No counterpart in the reference, whose planner
 * runs on the host after a device-to-host copy of every layer's routing
 * (dsv4_arena.py:68-127 over native/locali_core.c:259-313). These calls keep
 * the planner state in device memory and run locali_cache_plan_each's rules
 * (SLRU or LFU_DECAY, the previous demand call's slots pinned, every slot
 * resolved in a call pinned for the keys after it, the LFU token tick on
 * layer-0 calls of at most top_k experts) in one kernel per layer call, so
 * that a decode layer's router, planner, fills and expert kernels queue on
 * one stream with no host synchronisation.
 *
 * The state is one device buffer of locali_dplan_state_bytes() bytes,
 * 256-byte aligned, set up by locali_dplan_init on a stream. Keys are
 * layer * n_experts + expert, slot 0 is reserved, and usable slots are handed
 * out highest-first, as the host planner. The kernel holds the slot state in
 * LDS: locali_dplan_lds_bytes(slots, n_experts, policy) must stay within
 * 156 KiB (about 10,000 slots under SLRU and 5,600 under LFU_DECAY for 256
 * experts); locali_dplan_plan refuses larger ones.
 *
 * locali_dplan_plan plans the distinct experts of expert_idx[routes] (device
 * int32, values in [0, n_experts)) in first-appearance order for `layer`,
 * writes route_slot[routes] (device int32: each route's slot, 0 for a route
 * whose expert could not be placed), the call's fill list (its misses, in
 * order) and per-key results (locali_cache_result, as plan_each) into the
 * state. key_capacity, slots, policy and max_routes repeat the values given
 * to init (the kernel checks them against the state). Errors found on the
 * device do not stop the stream: they set a sticky code in the state
 * (LOCALI_DPLAN_E_*) that locali_dplan_read returns.
 *
 * locali_dplan_fill copies every miss of the state's last plan from pinned
 * host memory into its slot: host_src is a device array of key_capacity
 * device-visible addresses (locali_dplan_host_view), the expert's records
 * back to back in the order of dst_base; record a of an expert in slot s lands
 * at dst_base[a] + s * slot_bytes[a]. max_misses is an upper bound on the
 * misses (the plan call's routes); 0 launches nothing. The copy runs as a
 * persistent grid of 64 workgroups whatever the miss count. All of the
 * state's calls must run in stream order.
 *
 * locali_dplan_plan_fill is locali_dplan_plan followed by locali_dplan_fill
 * (the same decisions, route slots, results and copies) in one launch: the
 * planner workgroup publishes each miss in device memory as it decides it,
 * and 16 copy workgroups of the same grid start its copy meanwhile, so the
 * PCIe copy overlaps the planning of the keys after it and no launch
 * separates the two. The copy workgroups wait on the planner workgroup, which
 * is dispatched first; one that still waits after about a second gives up
 * and sets LOCALI_DPLAN_E_FILL.
 *
 * locali_dplan_prefetch is the cross-layer prefetch call of the same planner
 * (reference arena.py:518-541 over native/locali_core.c:259-313, as
 * V4ArenaStore.submit(..., prefetch=True) makes it on the host): expert_idx
 * and weights are `rows` rows of top_k routes of a lookahead routing (device
 * int32 and fp32); the call's keys are, row by row, each row's take_k highest
 * weights in descending order, equal weights in row order (every route in
 * route order when take_k is 0 or >= top_k), deduplicated in first-appearance
 * order. It plans them with hits left in place (touch_hits 0), the last
 * demand call's slots pinned and not replaced, no LFU token tick, and keys it
 * cannot place dropped without error; it writes no route slots, and counts
 * its placed misses as prefetched. A later demand hit on a slot a prefetch
 * filled counts as prefetch_used, its eviction before one as
 * prefetch_wasted. With dst_base non-null the launch also copies the placed
 * misses, as locali_dplan_plan_fill; with dst_base null it only plans
 * (locali_dplan_fill copies afterwards). It must run in stream order with the
 * state's other calls.
 *
 * locali_dplan_read copies the counters (and up to max_results per-key
 * results of the last call) to the host and waits for the stream.
 */
#define LOCALI_DPLAN_MAX_ARRAYS 16
#define LOCALI_DPLAN_MAX_EXPERTS 1024
enum {
    LOCALI_DPLAN_E_EXPERT = 1,   /* a route's expert outside [0, n_experts) */
    LOCALI_DPLAN_E_PLACE = 2,    /* a demanded key found no unpinned slot */
    LOCALI_DPLAN_E_CONFIG = 3,   /* plan arguments disagree with the state */
    LOCALI_DPLAN_E_FILL = 4,     /* a fused copy workgroup gave up waiting for the planner */
};

typedef struct {
    uint64_t hits, misses, evictions, calls;
    int32_t error;
    int32_t probation, protected_, free_slots;
    int32_t last_keys, last_misses;
    uint64_t prefetched, prefetch_used, prefetch_wasted;
} locali_dplan_stats;

size_t locali_dplan_state_bytes(int32_t key_capacity, int32_t slots, int32_t max_routes);
size_t locali_dplan_lds_bytes(int32_t slots, int32_t n_experts, int32_t policy);
int locali_dplan_init(void *state, size_t state_bytes, int32_t key_capacity, int32_t slots,
                      int32_t protected_capacity, int32_t policy, int32_t max_routes, void *stream);
int locali_dplan_plan(void *state, int32_t key_capacity, int32_t slots, int32_t policy, int32_t max_routes,
                      const int32_t *expert_idx, int32_t routes, int32_t layer, int32_t n_experts, int32_t top_k,
                      int32_t touch_hits, int32_t *route_slot, void *stream);
int locali_dplan_fill(const void *state, void *const *dst_base, const size_t *slot_bytes, int32_t n_arrays,
                      const uint64_t *host_src, int32_t layer, int32_t n_experts, int32_t max_misses,
                      void *stream);
int locali_dplan_plan_fill(void *state, int32_t key_capacity, int32_t slots, int32_t policy, int32_t max_routes,
                           const int32_t *expert_idx, int32_t routes, int32_t layer, int32_t n_experts,
                           int32_t top_k, int32_t touch_hits, int32_t *route_slot, void *const *dst_base,
                           const size_t *slot_bytes, int32_t n_arrays, const uint64_t *host_src, void *stream);
int locali_dplan_prefetch(void *state, int32_t key_capacity, int32_t slots, int32_t policy, int32_t max_routes,
                          const int32_t *expert_idx, const float *weights, int32_t rows, int32_t top_k,
                          int32_t take_k, int32_t layer, int32_t n_experts, void *const *dst_base,
                          const size_t *slot_bytes, int32_t n_arrays, const uint64_t *host_src, void *stream);
int locali_dplan_host_view(const void *const *src_host, int32_t n, uint64_t *out);
int locali_dplan_read(const void *state, locali_dplan_stats *stats, locali_cache_result *results,
                      int32_t max_results, void *stream);
int32_t locali_dplan_peek(const void *state, int32_t key, void *stream);

#ifdef __cplusplus
}
#endif

#endif
