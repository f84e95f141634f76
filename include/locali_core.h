/*
 * Host-side expert slot planner: segmented-LRU (SLRU) and LFU-with-decay
 * placement of (layer, expert) keys into a fixed pool of arena slots.
 *
 * Drop-in C ABI for Locali's native planner. Every declaration below has the
 * same name, argument meaning, return codes and struct layout as the
 * reference interface it replaces, so `locali_native.py`'s ctypes bindings
 * load this library unchanged:
 *
 *   locali_cache_result          native/locali_core.h:18-24   (16-byte record)
 *   locali_cache_create          native/locali_core.h:26-28   (-> locali_core.c:184-190)
 *   locali_cache_create_policy   native/locali_core.h:29-32   (-> locali_core.c:192-234)
 *   locali_cache_destroy         native/locali_core.h:33      (-> locali_core.c:236-248)
 *   locali_cache_note_token      native/locali_core.h:34      (-> locali_core.c:250-257)
 *   locali_cache_plan            native/locali_core.h:36-42   (-> locali_core.c:259-313)
 *   locali_cache_peek            native/locali_core.h:44      (-> locali_core.c:315-317)
 *   locali_cache_probation_size  native/locali_core.h:45      (-> locali_core.c:319-321)
 *   locali_cache_protected_size  native/locali_core.h:46      (-> locali_core.c:323-325)
 *
 * Semantics:
 *   - Slot 0 is reserved (the all-zero slot); usable slots are 1..slots-1 and a
 *     fresh planner hands them out highest-first.
 *   - SLRU: a miss enters probation; a hit with touch_hits promotes it to
 *     protected (or refreshes LRU order when protected_capacity == 0).
 *     Protected overflow demotes its LRU entry back to probation.
 *   - LFU_DECAY: every planned key gains one hotness unit and a clock stamp;
 *     the victim is the unpinned resident key with the lowest hotness, oldest
 *     stamp on ties; note_token halves every hotness each 16th call.
 *   - A slot listed in pinned_slots is never chosen as a victim in that call.
 *
 * Errors: create returns NULL on bad arguments (key_capacity <= 0, slots < 2,
 * protected_capacity < 0 or >= slots, unknown policy) or allocation failure.
 * plan returns 0 on success, -1 for a NULL cache / NULL arrays with a non-zero
 * count, -3 on the first out-of-range key (earlier results are written and the
 * planner state already reflects them). Not thread-safe: one caller thread per
 * planner. plan never allocates.
 */
#ifndef LOCALI_CORE_H
#define LOCALI_CORE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct locali_cache locali_cache;

enum {
    LOCALI_CACHE_SLRU = 0,
    LOCALI_CACHE_LFU_DECAY = 1,
};

typedef struct {
    int32_t key;
    int32_t slot;
    int32_t evicted_key;
    uint8_t hit;
    uint8_t placed;
} locali_cache_result;

locali_cache *locali_cache_create(int32_t key_capacity,
                                  int32_t slots,
                                  int32_t protected_capacity);
locali_cache *locali_cache_create_policy(int32_t key_capacity,
                                         int32_t slots,
                                         int32_t protected_capacity,
                                         int32_t policy);
void locali_cache_destroy(locali_cache *cache);
void locali_cache_note_token(locali_cache *cache);

int locali_cache_plan(locali_cache *cache,
                      const int32_t *keys,
                      size_t key_count,
                      const int32_t *pinned_slots,
                      size_t pinned_count,
                      int touch_hits,
                      locali_cache_result *results);

int32_t locali_cache_peek(const locali_cache *cache, int32_t key);
int32_t locali_cache_probation_size(const locali_cache *cache);
int32_t locali_cache_protected_size(const locali_cache *cache);

#ifdef __cplusplus
}
#endif

#endif
