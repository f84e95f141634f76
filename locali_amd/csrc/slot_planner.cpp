// Expert slot planner (host side). Exports the locali_cache_* C ABI declared in
// include/locali_core.h with the placement rules of the reference planner
// (native/locali_core.c:39-325); the data structures are this library's own.
//
// State per planner:
//   - two recency-ordered segments (probation, protected), each an intrusive
//     doubly linked list threaded through per-key link arrays, head = least
//     recently used;
//   - a stack of free slots (1..slots-1, popped from the top, so slots are
//     handed out highest-first);
//   - per-slot pin stamps compared against a per-call epoch, so pinning costs
//     O(pinned) per call and never needs a clear except on epoch wrap;
//   - LFU hotness counters and a logical clock.
// Everything is sized at creation; plan() never allocates.

#include "locali_core.h"
#include "locali_planner.h"

#include <algorithm>
#include <cstring>
#include <limits>
#include <new>
#include <vector>

namespace {

constexpr uint8_t kNowhere = 0;
constexpr uint8_t kProbation = 1;
constexpr uint8_t kProtected = 2;
constexpr int32_t kNil = -1;

struct Segment {
    int32_t head = kNil;   // least recently used
    int32_t tail = kNil;   // most recently used
    int32_t count = 0;
};

}  // namespace

struct locali_cache {
    int32_t n_keys = 0;
    int32_t n_slots = 0;
    int32_t policy = LOCALI_CACHE_SLRU;
    int32_t protected_cap = 0;
    int32_t probation_cap = 0;
    uint32_t tokens_seen = 0;
    uint32_t epoch = 0;
    uint64_t clock = 0;

    Segment seg[3];                      // indexed by kProbation / kProtected
    std::vector<int32_t> slot_of;        // key -> slot or kNil
    std::vector<int32_t> owner_of;       // slot -> key or kNil
    std::vector<int32_t> prev_link;      // key -> previous key in its segment
    std::vector<int32_t> next_link;      // key -> next key in its segment
    std::vector<uint8_t> where;          // key -> segment id
    std::vector<int32_t> free_stack;     // free slots, top = back
    std::vector<uint32_t> hot;           // LFU hotness
    std::vector<uint64_t> stamp;         // LFU recency stamp
    std::vector<uint32_t> pin_stamp;     // slot -> epoch it was pinned in

    bool key_ok(int32_t key) const { return key >= 0 && key < n_keys; }

    void unlink(int32_t key) {
        Segment &s = seg[where[key]];
        const int32_t p = prev_link[key];
        const int32_t n = next_link[key];
        (p == kNil ? s.head : next_link[p]) = n;
        (n == kNil ? s.tail : prev_link[n]) = p;
        prev_link[key] = next_link[key] = kNil;
        where[key] = kNowhere;
        --s.count;
    }

    void push_mru(int32_t key, uint8_t segment) {
        Segment &s = seg[segment];
        prev_link[key] = s.tail;
        next_link[key] = kNil;
        (s.tail == kNil ? s.head : next_link[s.tail]) = key;
        s.tail = key;
        where[key] = segment;
        ++s.count;
    }

    bool pinned(int32_t slot) const {
        return slot >= 0 && pin_stamp[slot] == epoch;
    }

    // Oldest key of a segment whose slot is not pinned this call.
    int32_t oldest_unpinned(uint8_t segment) const {
        for (int32_t k = seg[segment].head; k != kNil; k = next_link[k])
            if (!pinned(slot_of[k])) return k;
        return kNil;
    }

    // SLRU hit with touch: refresh protected, refresh plain LRU, or promote a
    // probation entry and demote protected overflow.
    void refresh(int32_t key) {
        const uint8_t from = where[key];
        unlink(key);
        if (from == kProtected || protected_cap == 0) {
            push_mru(key, from == kProtected ? kProtected : kProbation);
            return;
        }
        push_mru(key, kProtected);
        if (seg[kProtected].count > protected_cap) {
            const int32_t demoted = seg[kProtected].head;
            unlink(demoted);
            push_mru(demoted, kProbation);
        }
    }

    void bind(int32_t key, int32_t slot) {
        slot_of[key] = slot;
        owner_of[slot] = key;
        push_mru(key, kProbation);
    }

    int32_t evict(int32_t victim) {
        const int32_t slot = slot_of[victim];
        unlink(victim);
        slot_of[victim] = kNil;
        owner_of[slot] = kNil;
        return slot;
    }

    // SLRU miss. Probation has a fixed share of the slots: once it is full (or
    // nothing is free) its oldest unpinned entry is recycled; protected is
    // raided only when probation offers no victim.
    bool place_slru(int32_t key, int32_t *slot_out, int32_t *evicted_out) {
        const bool probation_full = seg[kProbation].count >= probation_cap;
        const bool have_free = !free_stack.empty();
        int32_t victim = kNil;
        if (probation_full || !have_free) victim = oldest_unpinned(kProbation);
        if (victim == kNil && !probation_full && have_free) {
            *slot_out = free_stack.back();
            free_stack.pop_back();
        } else {
            if (victim == kNil) victim = oldest_unpinned(kProtected);
            if (victim == kNil) return false;
            *evicted_out = victim;
            *slot_out = evict(victim);
        }
        bind(key, *slot_out);
        return true;
    }

    // Unpinned resident key with the lowest hotness; oldest stamp on ties.
    int32_t coldest_unpinned() const {
        int32_t best = kNil;
        uint32_t best_hot = std::numeric_limits<uint32_t>::max();
        uint64_t best_stamp = std::numeric_limits<uint64_t>::max();
        for (int32_t k = seg[kProbation].head; k != kNil; k = next_link[k]) {
            if (pinned(slot_of[k])) continue;
            if (hot[k] < best_hot || (hot[k] == best_hot && stamp[k] < best_stamp)) {
                best = k;
                best_hot = hot[k];
                best_stamp = stamp[k];
            }
        }
        return best;
    }

    bool place_lfu(int32_t key, int32_t *slot_out, int32_t *evicted_out) {
        if (!free_stack.empty()) {
            *slot_out = free_stack.back();
            free_stack.pop_back();
        } else {
            const int32_t victim = coldest_unpinned();
            if (victim == kNil) return false;
            *evicted_out = victim;
            *slot_out = evict(victim);
        }
        bind(key, *slot_out);
        return true;
    }
};

extern "C" {

locali_cache *locali_cache_create(int32_t key_capacity, int32_t slots,
                                  int32_t protected_capacity) {
    return locali_cache_create_policy(key_capacity, slots, protected_capacity,
                                      LOCALI_CACHE_SLRU);
}

locali_cache *locali_cache_create_policy(int32_t key_capacity, int32_t slots,
                                         int32_t protected_capacity,
                                         int32_t policy) {
    if (key_capacity <= 0 || slots < 2 || protected_capacity < 0 ||
        protected_capacity >= slots)
        return nullptr;
    if (policy != LOCALI_CACHE_SLRU && policy != LOCALI_CACHE_LFU_DECAY)
        return nullptr;
    // LFU keeps every resident key in one segment.
    if (policy == LOCALI_CACHE_LFU_DECAY) protected_capacity = 0;
    locali_cache *c = new (std::nothrow) locali_cache();
    if (!c) return nullptr;
    try {
        c->n_keys = key_capacity;
        c->n_slots = slots;
        c->policy = policy;
        c->protected_cap = protected_capacity;
        c->probation_cap = slots - 1 - protected_capacity;
        c->slot_of.assign(key_capacity, kNil);
        c->prev_link.assign(key_capacity, kNil);
        c->next_link.assign(key_capacity, kNil);
        c->where.assign(key_capacity, kNowhere);
        c->hot.assign(key_capacity, 0u);
        c->stamp.assign(key_capacity, 0u);
        c->owner_of.assign(slots, kNil);
        c->pin_stamp.assign(slots, 0u);
        c->free_stack.reserve(slots - 1);
        for (int32_t s = 1; s < slots; ++s) c->free_stack.push_back(s);
    } catch (const std::bad_alloc &) {
        delete c;
        return nullptr;
    }
    return c;
}

void locali_cache_destroy(locali_cache *cache) { delete cache; }

void locali_cache_note_token(locali_cache *cache) {
    if (!cache || cache->policy != LOCALI_CACHE_LFU_DECAY) return;
    if (++cache->tokens_seen % 16u != 0u) return;
    for (uint32_t &h : cache->hot) h >>= 1;
}

}  // extern "C"

namespace {

// plan() of the C ABI; with pin_resolved every slot a key resolves to (hit
// or placed) is pinned for the keys after it in the same call.
int plan_keys(locali_cache *cache, const int32_t *keys, size_t key_count, const int32_t *pinned_slots,
              size_t pinned_count, int touch_hits, locali_cache_result *results, bool pin_resolved) {
    if (!cache) return -1;
    if (key_count && (!keys || !results)) return -1;
    if (++cache->epoch == 0) {
        std::fill(cache->pin_stamp.begin(), cache->pin_stamp.end(), 0u);
        cache->epoch = 1;
    }
    for (size_t i = 0; i < pinned_count && pinned_slots; ++i) {
        const int32_t s = pinned_slots[i];
        if (s > 0 && s < cache->n_slots) cache->pin_stamp[s] = cache->epoch;
    }
    const bool lfu = cache->policy == LOCALI_CACHE_LFU_DECAY;
    for (size_t i = 0; i < key_count; ++i) {
        const int32_t key = keys[i];
        locali_cache_result r;
        std::memset(&r, 0, sizeof(r));
        r.key = key;
        r.slot = kNil;
        r.evicted_key = kNil;
        if (!cache->key_ok(key)) return -3;
        if (lfu) {
            if (cache->hot[key] != std::numeric_limits<uint32_t>::max())
                ++cache->hot[key];
            cache->stamp[key] = ++cache->clock;
        }
        const int32_t resident = cache->slot_of[key];
        if (resident != kNil) {
            r.hit = 1;
            r.placed = 1;
            r.slot = resident;
            if (touch_hits && !lfu) cache->refresh(key);
        } else {
            const bool ok = lfu ? cache->place_lfu(key, &r.slot, &r.evicted_key)
                                : cache->place_slru(key, &r.slot, &r.evicted_key);
            r.placed = ok ? 1 : 0;
        }
        results[i] = r;
        if (pin_resolved && r.placed && r.slot > 0 && r.slot < cache->n_slots) cache->pin_stamp[r.slot] = cache->epoch;
    }
    return 0;
}

}  // namespace

extern "C" {

int locali_cache_plan(locali_cache *cache, const int32_t *keys,
                      size_t key_count, const int32_t *pinned_slots,
                      size_t pinned_count, int touch_hits,
                      locali_cache_result *results) {
    return plan_keys(cache, keys, key_count, pinned_slots, pinned_count, touch_hits, results, false);
}

int locali_cache_plan_each(locali_cache *cache, const int32_t *keys, size_t key_count,
                           const int32_t *pinned_slots, size_t pinned_count, int touch_hits,
                           locali_cache_result *results) {
    return plan_keys(cache, keys, key_count, pinned_slots, pinned_count, touch_hits, results, true);
}

int32_t locali_cache_peek(const locali_cache *cache, int32_t key) {
    if (!cache || !cache->key_ok(key)) return kNil;
    return cache->slot_of[key];
}

int32_t locali_cache_probation_size(const locali_cache *cache) {
    return cache ? cache->seg[kProbation].count : -1;
}

int32_t locali_cache_protected_size(const locali_cache *cache) {
    return cache ? cache->seg[kProtected].count : -1;
}

}  // extern "C"
