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

#ifdef __cplusplus
}
#endif

#endif
