// Device-resident expert slot planner: the placement rules of
// locali_cache_plan_each (slot_planner.cpp; reference native/locali_core.c:
// 39-325 plus the per-key pinning of locali_planner.h), run by one
// workgroup per layer call over state kept in device memory, so that a
// layer's routing, placement, fills and expert kernels queue on one stream
// without a host round trip.
//
// Representation. The host planner threads each segment (probation,
// protected) as a doubly linked list in recency order; here every resident
// slot carries the stamp of its latest move to a segment's most recent end
// (one counter, incremented per move), so a segment's least recently used
// entry is the one with the smallest stamp, and "oldest unpinned entry of a
// segment" is an argmin over the slots that all 1024 threads take together.
// Pins are a per-call byte per slot. LFU hotness and stamps are per key, as
// in the host planner, with a per-slot copy for the victim search.
//
// One call (dplan_kernel): the slot arrays and this layer's keys are read
// into LDS; the routes' experts are deduplicated in first-appearance order;
// the previous call's slots are pinned; on layer 0 with at most top_k
// experts the LFU token tick runs (halving every hotness each 16th tick);
// then thread 0 plans the keys in order, each resolved slot pinned for the
// keys after it, and the workgroup joins it for every victim search; last,
// the slot of every route, the fill list (the call's misses) and the
// per-key results are written, and the slots the call changed go back to
// device memory.
//
// dplan_fill_kernel copies each miss of the last call from its pinned host
// payload (the expert's records back to back) into its slot, reading the
// host memory over PCIe itself, with a small persistent grid.
//
// The fused launch (dplan_kernel<true>) does both: workgroup 0 plans and
// publishes each miss in the state's header as soon as it is placed, and the
// copy workgroups behind it start that miss's copy while the planner decides
// the keys after it. On the 43-layer decode loop this moved the host-to-HBM
// rate from 44.8 to 45.5 GB/s against the planner and copy launched one
// after the other.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "locali_moe.h"
#include "locali_planner.h"

namespace locali {
int set_error(int code, const char *msg);
}

namespace {

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;
constexpr int kFillThreads = 256;
constexpr int kFillUnits = 8;                  // 16-byte units per thread
constexpr int kFillGrid = 64;                  // workgroups of the copy kernel (persistent)
constexpr int kFusedUnits = 8;                 // 16-byte units per thread of the fused copy workgroups
constexpr int kFusedCopiers = 16;              // copy workgroups of the fused kernel (2 MiB in flight)
// The fused kernel's publication word (DPlanHeader::pub): misses listed so
// far, and the closing bit once the list is final.
constexpr int32_t kPubCount = 0x3fffffff, kPubClosed = 0x40000000;
constexpr uint32_t kPubMaxSpins = 1u << 22;    // about a second of polling
constexpr uint8_t kNowhere = 0, kProbation = 1, kProtected = 2;
constexpr size_t kPlanMaxLds = 160 * 1024;
constexpr size_t kPlanMaxDynamicLds = kPlanMaxLds - 4096;   // the rest is the kernel's static LDS
constexpr size_t kDefaultLds = 64 * 1024;                   // per workgroup without the attribute

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct DPlanHeader {
    int32_t n_keys, n_slots, policy, protected_cap;
    int32_t probation_cap, max_routes, count_probation, count_protected;
    int32_t free_count, n_pinned, n_want, n_miss;
    int32_t error, tokens_seen, max_experts, pub;
    int32_t exited, pad[3];
    uint64_t rclock, lclock;
    uint64_t hits, misses, evictions, calls;
    uint64_t prefetched, pf_used, pf_wasted;
};

__host__ __device__ constexpr size_t align256(size_t x) { return (x + 255) & ~size_t{255}; }

struct DPlanLayout {
    size_t slot_of, hot, lst, owner, where, spf, rst, pinned, res, miss_e, miss_s, total;
};

__host__ __device__ inline DPlanLayout dplan_layout(int n_keys, int n_slots, int max_routes) {
    DPlanLayout L{};
    size_t off = align256(sizeof(DPlanHeader));
    auto take = [&off](size_t bytes) {
        const size_t at = off;
        off = align256(off + bytes);
        return at;
    };
    L.slot_of = take(sizeof(int32_t) * n_keys);
    L.hot = take(sizeof(uint32_t) * n_keys);
    L.lst = take(sizeof(uint64_t) * n_keys);
    L.owner = take(sizeof(int32_t) * n_slots);
    L.where = take(sizeof(uint8_t) * n_slots);
    L.spf = take(sizeof(uint8_t) * n_slots);
    L.rst = take(sizeof(uint64_t) * n_slots);
    L.pinned = take(sizeof(int32_t) * max_routes);
    L.res = take(sizeof(locali_cache_result) * max_routes);
    L.miss_e = take(sizeof(int32_t) * max_routes);
    L.miss_s = take(sizeof(int32_t) * max_routes);
    L.total = off;
    return L;
}

// Dynamic LDS of one plan call: slot-indexed state (recency stamps, LFU
// hotness and stamps for the LFU policy, owners, segments, pins, the flag of
// a slot whose key a prefetch placed and no demand call has used yet), then the
// layer's experts (their keys' slots, hotness and stamps, first route, slot
// chosen, the deduplicated list).
struct PlanLds {
    uint64_t *rst, *lst, *klst;
    uint32_t *hot, *khot;
    int32_t *owner, *kslot, *first, *eslot, *want;
    uint8_t *where, *pin, *dirty, *spf;
};

__host__ __device__ inline size_t plan_lds_bytes(int n_slots, int E, bool lfu) {
    size_t b = sizeof(uint64_t) * n_slots + sizeof(uint64_t) * E;       // rst, klst
    if (lfu) b += sizeof(uint64_t) * n_slots + sizeof(uint32_t) * n_slots;   // lst, hot
    b += sizeof(uint32_t) * E;                                            // khot
    b += sizeof(int32_t) * n_slots + 4 * sizeof(int32_t) * E;            // owner, kslot, first, eslot, want
    b += 4 * sizeof(uint8_t) * n_slots;                                   // where, pin, dirty, spf
    return (b + 15) & ~size_t{15};
}

__device__ inline PlanLds carve(unsigned char *p, int n_slots, int E, bool lfu) {
    PlanLds L{};
    auto take = [&p](size_t bytes) {
        unsigned char *at = p;
        p += bytes;
        return at;
    };
    L.rst = reinterpret_cast<uint64_t *>(take(sizeof(uint64_t) * n_slots));
    L.klst = reinterpret_cast<uint64_t *>(take(sizeof(uint64_t) * E));
    if (lfu) {
        L.lst = reinterpret_cast<uint64_t *>(take(sizeof(uint64_t) * n_slots));
        L.hot = reinterpret_cast<uint32_t *>(take(sizeof(uint32_t) * n_slots));
    }
    L.khot = reinterpret_cast<uint32_t *>(take(sizeof(uint32_t) * E));
    L.owner = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * n_slots));
    L.kslot = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * E));
    L.first = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * E));
    L.eslot = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * E));
    L.want = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * E));
    L.where = take(n_slots);
    L.pin = take(n_slots);
    L.dirty = take(n_slots);
    L.spf = take(n_slots);
    return L;
}

// Scan kinds: the oldest unpinned entry of probation / protected (SLRU
// victims), the oldest protected entry pinned or not (the demotion of
// protected overflow), the coldest unpinned entry (LFU victim: lowest
// hotness, then oldest LFU stamp).
enum ScanKind : int { kScanNone = 0, kScanProbation = 1, kScanProtected = 2, kScanProtectedAny = 3, kScanLfu = 4 };

struct PlanShared {
    int32_t kind1, kind2, result, n_want, decay, bad, avail, closed;
    int32_t wave_count[kPlanWaves];
    uint64_t red_a[kPlanWaves], red_b[kPlanWaves];
    int32_t red_s[kPlanWaves];
};

__device__ inline uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, 64);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, 64);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Lexicographic arg-min of (a, b, slot) over `lanes` lanes of the wave (a
// power of two), by butterfly; ties of (a, b) take the larger slot (only
// empty candidates tie: stamps are unique).
__device__ inline void argmin_lanes(uint64_t &a, uint64_t &b, int &s, int lanes) {
    for (int m = lanes / 2; m >= 1; m >>= 1) {
        const uint64_t oa = shfl_xor_u64(a, m), ob = shfl_xor_u64(b, m);
        const int os = __shfl_xor(s, m, 64);
        if (oa < a || (oa == a && (ob < b || (ob == b && os > s)))) {
            a = oa;
            b = ob;
            s = os;
        }
    }
}

// Victim search over slots 1 .. n_slots-1 by the whole workgroup; returns
// the slot (or -1) to every thread. Stamps are unique among resident slots,
// so the minimum is unique.
__device__ int scan_slots(const PlanLds &L, int n_slots, int kind, PlanShared &sh) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint8_t seg = (kind == kScanProtected || kind == kScanProtectedAny) ? kProtected : kProbation;
    const bool pin_filter = kind != kScanProtectedAny;
    uint64_t ba = ~uint64_t{0}, bb = ~uint64_t{0};
    int bs = -1;
    for (int s = 1 + tid; s < n_slots; s += kPlanThreads) {
        if (L.owner[s] < 0 || L.where[s] != seg || (pin_filter && L.pin[s])) continue;
        const uint64_t a = kind == kScanLfu ? uint64_t{L.hot[s]} : L.rst[s];
        const uint64_t b = kind == kScanLfu ? L.lst[s] : uint64_t{0};
        if (a < ba || (a == ba && b < bb)) {
            ba = a;
            bb = b;
            bs = s;
        }
    }
    argmin_lanes(ba, bb, bs, 64);
    if (lane == 0) {
        sh.red_a[wave] = ba;
        sh.red_b[wave] = bb;
        sh.red_s[wave] = bs;
    }
    __syncthreads();
    if (wave == 0) {
        // the waves' minima, one per lane
        ba = lane < kPlanWaves ? sh.red_a[lane] : ~uint64_t{0};
        bb = lane < kPlanWaves ? sh.red_b[lane] : ~uint64_t{0};
        bs = lane < kPlanWaves ? sh.red_s[lane] : -1;
        argmin_lanes(ba, bb, bs, kPlanWaves);
        if (lane == 0) sh.result = bs;
    }
    __syncthreads();
    return sh.result;
}

struct DPlanFillArgs {
    int32_t n_arrays;
    char *base[LOCALI_DPLAN_MAX_ARRAYS];
    uint64_t slot_bytes[LOCALI_DPLAN_MAX_ARRAYS];
    int64_t cum_units[LOCALI_DPLAN_MAX_ARRAYS + 1];   // 16-byte units before each array in the payload
};

// Copies chunk `chunk` (kThreads x kUnits 16-byte units) of an expert's
// payload at src into slot `slot` of the records in a.
template <int kThreads, int kUnits>
__device__ inline void copy_chunk(const DPlanFillArgs &a, const u32x4 *__restrict__ src, int slot, int64_t chunk,
                                  int64_t units) {
    const int64_t base = chunk * (kThreads * kUnits) + threadIdx.x;
    u32x4 v[kUnits];
#pragma unroll
    for (int i = 0; i < kUnits; ++i) {
        const int64_t u = base + static_cast<int64_t>(i) * kThreads;
        if (u < units) v[i] = __builtin_nontemporal_load(src + u);
    }
    // each record in turn (uniform), the thread's units that fall in it
    const int64_t first = base, last = base + static_cast<int64_t>(kUnits - 1) * kThreads;
    for (int j = 0; j < a.n_arrays; ++j) {
        const int64_t lo = a.cum_units[j], hi = a.cum_units[j + 1];
        if (hi <= first || lo > last) continue;
        u32x4 *dst = reinterpret_cast<u32x4 *>(a.base[j] + static_cast<int64_t>(slot) * a.slot_bytes[j]) - lo;
#pragma unroll
        for (int i = 0; i < kUnits; ++i) {
            const int64_t u = base + static_cast<int64_t>(i) * kThreads;
            if (u >= lo && u < hi && u < units) dst[u] = v[i];
        }
    }
}

// Every workgroup of the fused launch (the planner and each copy workgroup)
// counts its exit; the last one to leave sets the publication word back to
// zero for the next call. The planner counts too, so that a publication it
// makes after copy workgroups gave up waiting cannot outlive the launch.
__device__ inline void fused_exit(DPlanHeader *H) {
    const int before = __hip_atomic_fetch_add(&H->exited, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (before == static_cast<int>(gridDim.x) - 1) {
        __hip_atomic_store(&H->exited, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&H->pub, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// A copy workgroup of the fused kernel (blockIdx.x >= 1): chunks g, g + G,
// ... of the misses' payloads in list order, each once the planner
// workgroup has published its miss. Thread 0 polls the publication word and
// hands it to the workgroup through LDS, so the branch stays uniform; every
// workgroup leaves once the list is closed and its chunks are copied.
__device__ void copy_workgroup(unsigned char *state, const DPlanLayout &G, const DPlanFillArgs &a,
                               const uint64_t *__restrict__ host_src, int layer, int E, PlanShared &sh) {
    DPlanHeader *H = reinterpret_cast<DPlanHeader *>(state);
    const int32_t *miss_e = reinterpret_cast<const int32_t *>(state + G.miss_e);
    const int32_t *miss_s = reinterpret_cast<const int32_t *>(state + G.miss_s);
    const int64_t units = a.cum_units[a.n_arrays];
    constexpr int64_t kChunk = static_cast<int64_t>(kPlanThreads) * kFusedUnits;
    const int64_t chunks = (units + kChunk - 1) / kChunk;
    const int copiers = gridDim.x - 1;
    int avail = 0;
    bool closed = false;
    for (int64_t c = blockIdx.x - 1;; c += copiers) {
        const int64_t m = c / chunks;
        if (m >= avail && !closed) {
            if (threadIdx.x == 0) {
                int32_t p = 0;
                for (uint32_t spin = 0;; ++spin) {
                    p = __hip_atomic_load(&H->pub, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((p & kPubCount) > m || (p & kPubClosed)) break;
                    if (spin >= kPubMaxSpins) {   // the planner never closed: give up, marked
                        if (!H->error) H->error = LOCALI_DPLAN_E_FILL;
                        p |= kPubClosed;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(8);
                }
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                sh.avail = p & kPubCount;
                sh.closed = (p & kPubClosed) != 0;
            }
            __syncthreads();
            avail = sh.avail;
            closed = sh.closed != 0;
            __syncthreads();
        }
        if (m >= avail) break;
        const int mm = static_cast<int>(m);
        const int e = __hip_atomic_load(&miss_e[mm], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int slot = __hip_atomic_load(&miss_s[mm], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const u32x4 *src = reinterpret_cast<const u32x4 *>(host_src[static_cast<int64_t>(layer) * E + e]);
        if (src) copy_chunk<kPlanThreads, kFusedUnits>(a, src, slot, c % chunks, units);
    }
    __syncthreads();
    if (threadIdx.x == 0) fused_exit(H);
}

// Thread 0's planner state for one call (registers) and the list operations
// on the LDS copy; per-key arrays in device memory are written through.
struct Planner {
    const PlanLds &L;
    int32_t *g_slot_of;
    int layer, E, pcap, prob_cap;
    bool lfu, prefetch;
    int32_t n_probation, n_protected;
    int32_t free_count;
    uint64_t rclock, lclock;
    uint64_t pf_wasted = 0;

    __device__ Planner(const PlanLds &lds) : L(lds) {}

    // every change of a slot's owner, segment or stamp goes through these
    // two, which mark the slot for the write-back
    __device__ void unlink(int s) {
        if (L.where[s] == kProbation) --n_probation;
        else if (L.where[s] == kProtected) --n_protected;
        L.where[s] = kNowhere;
        L.dirty[s] = 1;
    }
    __device__ void push(int s, uint8_t seg) {
        L.dirty[s] = 1;
        L.where[s] = seg;
        L.rst[s] = ++rclock;
        if (seg == kProbation) ++n_probation;
        else ++n_protected;
    }
    __device__ void bind(int e, int key, int s) {
        L.kslot[e] = s;
        g_slot_of[key] = s;
        L.owner[s] = key;
        L.spf[s] = prefetch ? 1 : 0;
        push(s, kProbation);
        if (lfu) {
            L.hot[s] = L.khot[e];
            L.lst[s] = L.klst[e];
        }
    }
    // Frees slot v of its key; returns that key.
    __device__ int evict(int v) {
        const int k = L.owner[v];
        if (L.spf[v]) {   // a prefetched key leaves unused
            ++pf_wasted;
            L.spf[v] = 0;
        }
        unlink(v);
        g_slot_of[k] = -1;
        if (k >= layer * E && k < layer * E + E) L.kslot[k - layer * E] = -1;
        L.owner[v] = -1;
        return k;
    }
};

// The keys of a call, in order. A demand call takes its routes' experts in
// route order. A prefetch call reads rows of top_k routes with their gate
// weights and takes, row by row, the `take` highest weights of each row in
// descending order, equal weights in row order (a stable sort of the negated
// weights); with take >= top_k it takes every route in route order.
struct KeySeq {
    const int32_t *idx;
    const float *w;
    int top_k, take;
    bool ranked;

    __device__ int at(int p) const {
        if (!ranked) return idx[p];
        const int row = p / take, q = p - row * take;
        const int32_t *ri = idx + static_cast<int64_t>(row) * top_k;
        const float *rw = w + static_cast<int64_t>(row) * top_k;
        for (int j = 0; j < top_k; ++j) {
            const float wj = rw[j];
            int rank = 0;
            for (int i = 0; i < top_k; ++i) {
                const float wi = rw[i];
                rank += (wi > wj || (wi == wj && i < j)) ? 1 : 0;
            }
            if (rank == q) return ri[j];
        }
        return -1;   // NaN weights rank nowhere: the call is marked (LOCALI_DPLAN_E_EXPERT)
    }
};

// The planner's shape travels in the arguments (the launch sized its LDS by
// them); a state whose header disagrees is left alone and marked. A
// prefetch call (prefetch != 0; idx and weights are rows of top_k routes)
// plans its keys with hits left in place, does not replace the pinned set
// of the last demand call, skips the LFU token tick, drops keys it cannot
// place, writes no route slots and counts its placements as prefetched
// instead of hits and misses. kFused:
// workgroup 0 plans and publishes each miss as it is decided, workgroups 1..
// copy the published misses meanwhile (copy_workgroup).
template <bool kFused>
__global__ __launch_bounds__(kPlanThreads) void dplan_kernel(unsigned char *__restrict__ state, int n_keys,
                                                             int n_slots, int policy, int max_routes,
                                                             const int32_t *__restrict__ idx, int routes,
                                                             int layer, int E, int top_k, int touch_hits,
                                                             int32_t *__restrict__ route_slot, DPlanFillArgs fa,
                                                             const uint64_t *__restrict__ host_src,
                                                             const float *__restrict__ pf_weights, int take_k,
                                                             int prefetch) {
    extern __shared__ __align__(16) unsigned char plds[];
    __shared__ PlanShared sh;
    DPlanHeader *H = reinterpret_cast<DPlanHeader *>(state);
    const int tid = threadIdx.x;
    const DPlanLayout G = dplan_layout(n_keys, n_slots, max_routes);
    if (kFused && blockIdx.x > 0) {
        copy_workgroup(state, G, fa, host_src, layer, E, sh);
        return;
    }
    if (H->n_keys != n_keys || H->n_slots != n_slots || H->policy != policy || H->max_routes != max_routes) {
        if (tid == 0) {
            if (!H->error) H->error = LOCALI_DPLAN_E_CONFIG;
            if (kFused) {
                __hip_atomic_store(&H->pub, kPubClosed, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                fused_exit(H);
            }
        }
        return;
    }
    const bool lfu = policy == LOCALI_CACHE_LFU_DECAY;
    int32_t *g_slot_of = reinterpret_cast<int32_t *>(state + G.slot_of);
    uint32_t *g_hot = reinterpret_cast<uint32_t *>(state + G.hot);
    uint64_t *g_lst = reinterpret_cast<uint64_t *>(state + G.lst);
    int32_t *g_owner = reinterpret_cast<int32_t *>(state + G.owner);
    uint8_t *g_where = state + G.where;
    uint8_t *g_spf = state + G.spf;
    uint64_t *g_rst = reinterpret_cast<uint64_t *>(state + G.rst);
    int32_t *g_pinned = reinterpret_cast<int32_t *>(state + G.pinned);
    locali_cache_result *g_res = reinterpret_cast<locali_cache_result *>(state + G.res);
    int32_t *g_miss_e = reinterpret_cast<int32_t *>(state + G.miss_e);
    int32_t *g_miss_s = reinterpret_cast<int32_t *>(state + G.miss_s);
    const PlanLds L = carve(plds, n_slots, E, lfu);
    const int kbase = layer * E;
    const int take = prefetch && take_k > 0 && take_k < top_k ? take_k : top_k;
    const KeySeq seq{idx, pf_weights, top_k, take, take < top_k};
    const int n_seq = take < top_k ? routes / top_k * take : routes;

    // ---- state into LDS; the first keys and pins travel with it
    const int n_pinned_prev = H->n_pinned;
    const int my_e = tid < n_seq ? seq.at(tid) : -1;
    const int my_pin = tid < n_pinned_prev ? g_pinned[tid] : 0;
    for (int s = tid; s < n_slots; s += kPlanThreads) {
        const int k = g_owner[s];
        L.owner[s] = k;
        L.where[s] = g_where[s];
        L.spf[s] = g_spf[s];
        L.rst[s] = g_rst[s];
        L.pin[s] = 0;
        L.dirty[s] = 0;
        if (lfu) {
            L.hot[s] = k >= 0 ? g_hot[k] : 0u;
            L.lst[s] = k >= 0 ? g_lst[k] : uint64_t{0};
        }
    }
    for (int e = tid; e < E; e += kPlanThreads) {
        L.kslot[e] = g_slot_of[kbase + e];
        L.khot[e] = g_hot[kbase + e];
        L.klst[e] = g_lst[kbase + e];
        L.first[e] = INT_MAX;
        L.eslot[e] = 0;
    }
    if (tid == 0) sh.bad = 0;
    __syncthreads();

    // ---- the call's experts in first-appearance order; the previous
    // demand call's slots pinned
    for (int r = tid; r < n_seq; r += kPlanThreads) {
        const int e = r < kPlanThreads ? my_e : seq.at(r);
        if (e >= 0 && e < E) atomicMin(&L.first[e], r);
        else sh.bad = 1;
    }
    for (int j = tid; j < n_pinned_prev; j += kPlanThreads) {
        const int s = j < kPlanThreads ? my_pin : g_pinned[j];
        if (s > 0 && s < n_slots) L.pin[s] = 1;
    }
    __syncthreads();
    int carry = 0;
    for (int r0 = 0; r0 < n_seq; r0 += kPlanThreads) {
        const int r = r0 + tid;
        int e = -1;
        bool head = false;
        if (r < n_seq) {
            e = r0 == 0 ? my_e : seq.at(r);
            head = e >= 0 && e < E && L.first[e] == r;
        }
        const uint64_t m = __ballot(head);
        const int lane = tid & 63, wave = tid >> 6;
        if (lane == 0) sh.wave_count[wave] = __popcll(m);
        __syncthreads();
        int before = carry;
        for (int w = 0; w < wave; ++w) before += sh.wave_count[w];
        if (head) L.want[before + __popcll(m & ((uint64_t{1} << lane) - 1))] = e;
        int total = 0;
        for (int w = 0; w < kPlanWaves; ++w) total += sh.wave_count[w];
        carry += total;
        __syncthreads();
    }
    if (tid == 0) {
        sh.n_want = carry;
        int decay = 0;
        if (lfu && !prefetch && layer == 0 && carry <= top_k) {
            const uint32_t t = static_cast<uint32_t>(H->tokens_seen) + 1u;
            H->tokens_seen = static_cast<int32_t>(t);
            decay = t % 16u == 0u;
        }
        sh.decay = decay;
    }
    __syncthreads();
    if (sh.decay) {
        // the token tick before the call's keys (locali_cache_note_token)
        for (int k = tid; k < n_keys; k += kPlanThreads) g_hot[k] >>= 1;
        for (int s = tid; s < n_slots; s += kPlanThreads) L.hot[s] >>= 1;
        for (int e = tid; e < E; e += kPlanThreads) L.khot[e] >>= 1;
        __threadfence();
        __syncthreads();
    }

    // ---- the keys in order
    const int n_want = sh.n_want;
    Planner P(L);
    P.g_slot_of = g_slot_of;
    P.layer = layer;
    P.E = E;
    P.lfu = lfu;
    P.prefetch = prefetch != 0;
    P.pcap = H->protected_cap;
    P.prob_cap = H->probation_cap;
    P.n_probation = H->count_probation;
    P.n_protected = H->count_protected;
    P.free_count = H->free_count;
    P.rclock = H->rclock;
    P.lclock = H->lclock;
    enum Phase { kDone, kDemote, kLfuVictim, kSlruProbation, kSlruProtected };
    int phase = kDone, e = 0, key = 0, slot = -1, evicted = -1, hit = 0, placed = 0;
    bool prob_full = false, have_free = false;
    int n_pin = 0, n_miss = 0, fails = 0;
    uint64_t hits = 0, misses = 0, evictions = 0, pf_used = 0;
    for (int i = 0; i < n_want; ++i) {
        if (tid == 0) {
            e = L.want[i];
            key = kbase + e;
            phase = kDone;
            slot = -1;
            evicted = -1;
            hit = placed = 0;
            int kind = kScanNone;
            if (lfu) {
                uint32_t h = L.khot[e];
                if (h != UINT_MAX) ++h;
                L.khot[e] = h;
                g_hot[key] = h;
                const uint64_t st = ++P.lclock;
                L.klst[e] = st;
                g_lst[key] = st;
                const int s0 = L.kslot[e];
                if (s0 >= 0) {
                    L.hot[s0] = h;
                    L.lst[s0] = st;
                }
            }
            const int s0 = L.kslot[e];
            if (s0 >= 0) {
                hit = placed = 1;
                slot = s0;
                if (!prefetch && L.spf[s0]) {   // a demand call uses a prefetched key
                    ++pf_used;
                    L.spf[s0] = 0;
                    L.dirty[s0] = 1;
                }
                if (touch_hits && !lfu) {
                    const uint8_t from = L.where[s0];
                    P.unlink(s0);
                    if (from == kProtected || P.pcap == 0) {
                        P.push(s0, from == kProtected ? kProtected : kProbation);
                    } else {
                        P.push(s0, kProtected);
                        if (P.n_protected > P.pcap) {
                            kind = kScanProtectedAny;
                            phase = kDemote;
                        }
                    }
                }
            } else if (lfu) {
                if (P.free_count > 0) {
                    slot = P.free_count--;
                    P.bind(e, key, slot);
                    placed = 1;
                } else {
                    kind = kScanLfu;
                    phase = kLfuVictim;
                }
            } else {
                prob_full = P.n_probation >= P.prob_cap;
                have_free = P.free_count > 0;
                if (prob_full || !have_free) {
                    kind = kScanProbation;
                    phase = kSlruProbation;
                } else {
                    slot = P.free_count--;
                    P.bind(e, key, slot);
                    placed = 1;
                }
            }
            sh.kind1 = kind;
        }
        __syncthreads();
        const int kind1 = sh.kind1;
        const int r1 = kind1 != kScanNone ? scan_slots(L, n_slots, kind1, sh) : -1;
        if (tid == 0) {
            int kind = kScanNone;
            if (phase == kDemote) {
                if (r1 >= 0) {   // protected holds at least two entries here
                    P.unlink(r1);
                    P.push(r1, kProbation);
                }
                phase = kDone;
            } else if (phase == kLfuVictim) {
                if (r1 >= 0) {
                    evicted = P.evict(r1);
                    slot = r1;
                    P.bind(e, key, slot);
                    placed = 1;
                }
                phase = kDone;
            } else if (phase == kSlruProbation) {
                if (r1 < 0 && !prob_full && have_free) {
                    slot = P.free_count--;
                    P.bind(e, key, slot);
                    placed = 1;
                    phase = kDone;
                } else if (r1 >= 0) {
                    evicted = P.evict(r1);
                    slot = r1;
                    P.bind(e, key, slot);
                    placed = 1;
                    phase = kDone;
                } else {
                    kind = kScanProtected;
                    phase = kSlruProtected;
                }
            }
            sh.kind2 = kind;
        }
        __syncthreads();
        const int kind2 = sh.kind2;
        const int r2 = kind2 != kScanNone ? scan_slots(L, n_slots, kind2, sh) : -1;
        if (tid == 0) {
            if (phase == kSlruProtected && r2 >= 0) {
                evicted = P.evict(r2);
                slot = r2;
                P.bind(e, key, slot);
                placed = 1;
            }
            locali_cache_result res;
            res.key = key;
            res.slot = placed ? slot : -1;
            res.evicted_key = evicted;
            res.hit = static_cast<uint8_t>(hit);
            res.placed = static_cast<uint8_t>(placed);
            g_res[i] = res;
            if (placed) {
                L.eslot[e] = slot;
                L.pin[slot] = 1;
                if (!prefetch) g_pinned[n_pin++] = slot;
                if (!hit) {
                    g_miss_e[n_miss] = e;
                    g_miss_s[n_miss] = slot;
                    ++n_miss;
                    if (kFused) __hip_atomic_store(&H->pub, n_miss, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else {
                ++fails;
            }
            if (hit) ++hits;
            else ++misses;
            if (evicted >= 0) ++evictions;
        }
        __syncthreads();
    }

    // ---- outputs and state back to device memory; the fill list is final
    if (kFused && tid == 0) {
        __hip_atomic_store(&H->pub, n_miss | kPubClosed, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!prefetch) {
        for (int r = tid; r < routes; r += kPlanThreads) {
            const int x = idx[r];
            route_slot[r] = (x >= 0 && x < E) ? L.eslot[x] : 0;
        }
    }
    for (int s = tid; s < n_slots; s += kPlanThreads) {
        if (!L.dirty[s]) continue;   // only the slots this call changed
        g_owner[s] = L.owner[s];
        g_where[s] = L.where[s];
        g_spf[s] = L.spf[s];
        g_rst[s] = L.rst[s];
    }
    if (tid == 0) {
        H->count_probation = P.n_probation;
        H->count_protected = P.n_protected;
        H->free_count = P.free_count;
        H->rclock = P.rclock;
        H->lclock = P.lclock;
        if (!prefetch) H->n_pinned = n_pin;
        H->n_want = n_want;
        H->n_miss = n_miss;
        if (prefetch) {
            H->prefetched += n_miss;
        } else {
            H->hits += hits;
            H->misses += misses;
        }
        H->pf_used += pf_used;
        H->pf_wasted += P.pf_wasted;
        H->evictions += evictions;
        H->calls += 1;
        if (sh.bad && !H->error) H->error = LOCALI_DPLAN_E_EXPERT;
        if (fails && !prefetch && !H->error) H->error = LOCALI_DPLAN_E_PLACE;
        if (kFused) fused_exit(H);
    }
}

__global__ __launch_bounds__(256) void dplan_init_kernel(unsigned char *__restrict__ state, int n_keys, int n_slots,
                                                         int protected_cap, int policy, int max_routes) {
    const DPlanLayout G = dplan_layout(n_keys, n_slots, max_routes);
    int32_t *slot_of = reinterpret_cast<int32_t *>(state + G.slot_of);
    uint32_t *hot = reinterpret_cast<uint32_t *>(state + G.hot);
    uint64_t *lst = reinterpret_cast<uint64_t *>(state + G.lst);
    int32_t *owner = reinterpret_cast<int32_t *>(state + G.owner);
    uint8_t *where = state + G.where;
    uint8_t *spf = state + G.spf;
    uint64_t *rst = reinterpret_cast<uint64_t *>(state + G.rst);
    const int stride = gridDim.x * blockDim.x;
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < n_keys; k += stride) {
        slot_of[k] = -1;
        hot[k] = 0u;
        lst[k] = 0u;
    }
    for (int s = blockIdx.x * blockDim.x + threadIdx.x; s < n_slots; s += stride) {
        owner[s] = -1;
        where[s] = kNowhere;
        spf[s] = 0;
        rst[s] = 0u;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        DPlanHeader h{};
        h.n_keys = n_keys;
        h.n_slots = n_slots;
        h.policy = policy;
        h.protected_cap = protected_cap;
        h.probation_cap = n_slots - 1 - protected_cap;
        h.max_routes = max_routes;
        h.free_count = n_slots - 1;
        *reinterpret_cast<DPlanHeader *>(state) = h;
    }
}

// A persistent grid of kFillGrid workgroups: workgroup g takes chunks g,
// g + kFillGrid, ... of the misses' payloads (kFillThreads x kFillUnits
// 16-byte units each), which keeps enough host reads in flight for the PCIe
// link without a grid sized by the payload.
__global__ __launch_bounds__(kFillThreads) void dplan_fill_kernel(const unsigned char *__restrict__ state,
                                                                  DPlanFillArgs a,
                                                                  const uint64_t *__restrict__ host_src, int layer,
                                                                  int E) {
    const DPlanHeader *H = reinterpret_cast<const DPlanHeader *>(state);
    const int n_miss = H->n_miss;
    const DPlanLayout G = dplan_layout(H->n_keys, H->n_slots, H->max_routes);
    const int32_t *miss_e = reinterpret_cast<const int32_t *>(state + G.miss_e);
    const int32_t *miss_s = reinterpret_cast<const int32_t *>(state + G.miss_s);
    const int64_t units = a.cum_units[a.n_arrays];
    constexpr int64_t kChunk = static_cast<int64_t>(kFillThreads) * kFillUnits;
    const int64_t chunks = (units + kChunk - 1) / kChunk;
    for (int64_t c = blockIdx.x; c < n_miss * chunks; c += gridDim.x) {
        const int m = static_cast<int>(c / chunks);
        const u32x4 *src = reinterpret_cast<const u32x4 *>(host_src[static_cast<int64_t>(layer) * E + miss_e[m]]);
        if (src) copy_chunk<kFillThreads, kFillUnits>(a, src, miss_s[m], c % chunks, units);
    }
}

int dfail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int dfail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return locali::set_error(code, buf);
}

int dhip(hipError_t e, const char *where) {
    return dfail(LOCALI_E_HIP, "%s: %s", where, hipGetErrorString(e));
}

// The records' table of a fill: 16-byte aligned bases and slot sizes, and
// each record's first unit in an expert's payload.
int fill_args(void *const *dst_base, const size_t *slot_bytes, int32_t n_arrays, DPlanFillArgs *a,
              const char *who) {
    if (!dst_base || !slot_bytes || n_arrays < 1 || n_arrays > LOCALI_DPLAN_MAX_ARRAYS)
        return dfail(LOCALI_E_ARG, "%s: bad record table", who);
    a->n_arrays = n_arrays;
    for (int32_t i = 0; i < n_arrays; ++i) {
        if (!dst_base[i] || slot_bytes[i] % 16 || reinterpret_cast<uintptr_t>(dst_base[i]) % 16)
            return dfail(LOCALI_E_ARG, "%s: array %d not 16-byte aligned", who, i);
        a->base[i] = static_cast<char *>(dst_base[i]);
        a->slot_bytes[i] = slot_bytes[i];
        a->cum_units[i + 1] = a->cum_units[i] + static_cast<int64_t>(slot_bytes[i] / 16);
    }
    if (a->cum_units[n_arrays] < 1) return dfail(LOCALI_E_ARG, "%s: empty payload", who);
    return 0;
}

// The prefetch form of a call: the rows' gate weights and how many of each
// row's highest to take (0: every route).
struct PrefetchArgs {
    const float *weights = nullptr;
    int32_t take_k = 0;
    bool on = false;
};

// One planner launch: a single workgroup, or (fused) the planner workgroup
// and kFusedCopiers copy workgroups.
int plan_launch(bool fused, void *state, int32_t key_capacity, int32_t slots, int32_t policy, int32_t max_routes,
                const int32_t *expert_idx, int32_t routes, int32_t layer, int32_t n_experts, int32_t top_k,
                int32_t touch_hits, int32_t *route_slot, const DPlanFillArgs &fa, const uint64_t *host_src,
                void *stream, const PrefetchArgs &pf = PrefetchArgs{}) {
    if (routes == 0) return 0;
    if (!state || !expert_idx || (!route_slot && !pf.on) || routes < 0 || routes > max_routes || n_experts < 1 ||
        n_experts > LOCALI_DPLAN_MAX_EXPERTS || layer < 0 || top_k < 1)
        return dfail(LOCALI_E_ARG, "dplan_plan: bad arguments");
    if (pf.on && (routes % top_k || pf.take_k < 0 || (pf.take_k > 0 && pf.take_k < top_k && !pf.weights)))
        return dfail(LOCALI_E_ARG, "dplan_prefetch: bad arguments");
    if (static_cast<int64_t>(layer + 1) * n_experts > key_capacity)
        return dfail(LOCALI_E_ARG, "dplan_plan: layer %d x %d experts outside %d keys", layer, n_experts,
                     key_capacity);
    if (slots < 2 || key_capacity < 1 || max_routes < 1 ||
        (policy != LOCALI_CACHE_SLRU && policy != LOCALI_CACHE_LFU_DECAY))
        return dfail(LOCALI_E_ARG, "dplan_plan: bad planner shape");
    const size_t lds = plan_lds_bytes(slots, n_experts, policy == LOCALI_CACHE_LFU_DECAY);
    if (lds > kPlanMaxDynamicLds)
        return dfail(LOCALI_E_ARG, "dplan_plan: %d slots need %zu bytes of LDS; at most %zu", slots, lds,
                     kPlanMaxDynamicLds);
    // Above the default 64 KiB per workgroup the kernels need the larger
    // LDS allowance (gfx950: 160 KiB); requested once per kernel, and only by
    // a state that needs it, so that small states run wherever 64 KiB do.
    if (lds + (kPlanMaxLds - kPlanMaxDynamicLds) > kDefaultLds) {
        // the device's own per-workgroup limit first: on a part with less LDS
        // than gfx950's the call fails here with the figures, not at launch
        int dev = 0, optin = 0;
        hipError_t qe = hipGetDevice(&dev);
        if (qe == hipSuccess) qe = hipDeviceGetAttribute(&optin, hipDeviceAttributeSharedMemPerBlockOptin, dev);
        if (qe != hipSuccess) return dhip(qe, "dplan_plan LDS limit query");
        if (lds + (kPlanMaxLds - kPlanMaxDynamicLds) > static_cast<size_t>(optin))
            return dfail(LOCALI_E_ARG, "dplan_plan: %d slots need %zu bytes of LDS; this device allows %d per workgroup",
                         slots, lds + (kPlanMaxLds - kPlanMaxDynamicLds), optin);
        static const hipError_t attr0 = hipFuncSetAttribute(reinterpret_cast<const void *>(&dplan_kernel<false>),
                                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                                            static_cast<int>(kPlanMaxDynamicLds));
        static const hipError_t attr1 = hipFuncSetAttribute(reinterpret_cast<const void *>(&dplan_kernel<true>),
                                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                                            static_cast<int>(kPlanMaxDynamicLds));
        const hipError_t attr = fused ? attr1 : attr0;
        if (attr != hipSuccess) return dhip(attr, "dplan_plan attribute (LDS beyond 64 KiB per workgroup)");
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    unsigned char *sp = static_cast<unsigned char *>(state);
    if (fused)
        hipLaunchKernelGGL(dplan_kernel<true>, dim3(1 + kFusedCopiers), dim3(kPlanThreads), lds, st, sp, key_capacity,
                           slots, policy, max_routes, expert_idx, routes, layer, n_experts, top_k,
                           touch_hits ? 1 : 0, route_slot, fa, host_src, pf.weights, pf.take_k, pf.on ? 1 : 0);
    else
        hipLaunchKernelGGL(dplan_kernel<false>, dim3(1), dim3(kPlanThreads), lds, st, sp, key_capacity, slots,
                           policy, max_routes, expert_idx, routes, layer, n_experts, top_k, touch_hits ? 1 : 0,
                           route_slot, fa, host_src, pf.weights, pf.take_k, pf.on ? 1 : 0);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? dhip(e, "dplan_plan launch") : 0;
}

}  // namespace

extern "C" {

size_t locali_dplan_state_bytes(int32_t key_capacity, int32_t slots, int32_t max_routes) {
    if (key_capacity <= 0 || slots < 2 || max_routes < 1) return 0;
    return dplan_layout(key_capacity, slots, max_routes).total;
}

size_t locali_dplan_lds_bytes(int32_t slots, int32_t n_experts, int32_t policy) {
    return plan_lds_bytes(slots, n_experts, policy == LOCALI_CACHE_LFU_DECAY);
}

int locali_dplan_init(void *state, size_t state_bytes, int32_t key_capacity, int32_t slots,
                      int32_t protected_capacity, int32_t policy, int32_t max_routes, void *stream) {
    if (!state || key_capacity <= 0 || slots < 2 || protected_capacity < 0 || protected_capacity >= slots ||
        max_routes < 1)
        return dfail(LOCALI_E_ARG, "dplan_init: bad arguments");
    if (policy != LOCALI_CACHE_SLRU && policy != LOCALI_CACHE_LFU_DECAY)
        return dfail(LOCALI_E_ARG, "dplan_init: unknown policy %d", policy);
    if (policy == LOCALI_CACHE_LFU_DECAY) protected_capacity = 0;   // LFU keeps one segment
    if (reinterpret_cast<uintptr_t>(state) % 256)
        return dfail(LOCALI_E_ARG, "dplan_init: state must be 256-byte aligned");
    if (state_bytes < locali_dplan_state_bytes(key_capacity, slots, max_routes))
        return dfail(LOCALI_E_WORKSPACE, "dplan_init: state of %zu bytes, %zu needed", state_bytes,
                     locali_dplan_state_bytes(key_capacity, slots, max_routes));
    hipLaunchKernelGGL(dplan_init_kernel, dim3(64), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<unsigned char *>(state), key_capacity, slots, protected_capacity, policy,
                       max_routes);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? dhip(e, "dplan_init launch") : 0;
}

int locali_dplan_plan(void *state, int32_t key_capacity, int32_t slots, int32_t policy, int32_t max_routes,
                      const int32_t *expert_idx, int32_t routes, int32_t layer, int32_t n_experts, int32_t top_k,
                      int32_t touch_hits, int32_t *route_slot, void *stream) {
    return plan_launch(false, state, key_capacity, slots, policy, max_routes, expert_idx, routes, layer, n_experts,
                       top_k, touch_hits, route_slot, DPlanFillArgs{}, nullptr, stream);
}

int locali_dplan_fill(const void *state, void *const *dst_base, const size_t *slot_bytes, int32_t n_arrays,
                      const uint64_t *host_src, int32_t layer, int32_t n_experts, int32_t max_misses,
                      void *stream) {
    if (max_misses == 0) return 0;
    if (!state || !host_src || max_misses < 0 || layer < 0 || n_experts < 1)
        return dfail(LOCALI_E_ARG, "dplan_fill: bad arguments");
    DPlanFillArgs a{};
    if (const int rc = fill_args(dst_base, slot_bytes, n_arrays, &a, "dplan_fill")) return rc;
    hipLaunchKernelGGL(dplan_fill_kernel, dim3(kFillGrid), dim3(kFillThreads), 0, static_cast<hipStream_t>(stream),
                       static_cast<const unsigned char *>(state), a, host_src, layer, n_experts);
    const hipError_t e = hipGetLastError();
    return e != hipSuccess ? dhip(e, "dplan_fill launch") : 0;
}

int locali_dplan_plan_fill(void *state, int32_t key_capacity, int32_t slots, int32_t policy, int32_t max_routes,
                           const int32_t *expert_idx, int32_t routes, int32_t layer, int32_t n_experts,
                           int32_t top_k, int32_t touch_hits, int32_t *route_slot, void *const *dst_base,
                           const size_t *slot_bytes, int32_t n_arrays, const uint64_t *host_src, void *stream) {
    if (routes == 0) return 0;
    if (!host_src) return dfail(LOCALI_E_ARG, "dplan_plan_fill: bad arguments");
    DPlanFillArgs a{};
    if (const int rc = fill_args(dst_base, slot_bytes, n_arrays, &a, "dplan_plan_fill")) return rc;
    return plan_launch(true, state, key_capacity, slots, policy, max_routes, expert_idx, routes, layer, n_experts,
                       top_k, touch_hits, route_slot, a, host_src, stream);
}

int locali_dplan_prefetch(void *state, int32_t key_capacity, int32_t slots, int32_t policy, int32_t max_routes,
                          const int32_t *expert_idx, const float *weights, int32_t rows, int32_t top_k,
                          int32_t take_k, int32_t layer, int32_t n_experts, void *const *dst_base,
                          const size_t *slot_bytes, int32_t n_arrays, const uint64_t *host_src, void *stream) {
    if (rows == 0) return 0;
    if (rows < 0 || top_k < 1 || static_cast<int64_t>(rows) * top_k > max_routes)
        return dfail(LOCALI_E_ARG, "dplan_prefetch: bad arguments");
    PrefetchArgs pf;
    pf.weights = weights;
    pf.take_k = take_k;
    pf.on = true;
    const bool fused = dst_base != nullptr;
    DPlanFillArgs a{};
    if (fused) {
        if (!host_src) return dfail(LOCALI_E_ARG, "dplan_prefetch: bad arguments");
        if (const int rc = fill_args(dst_base, slot_bytes, n_arrays, &a, "dplan_prefetch")) return rc;
    }
    return plan_launch(fused, state, key_capacity, slots, policy, max_routes, expert_idx, rows * top_k, layer,
                       n_experts, top_k, 0, nullptr, a, host_src, stream, pf);
}

int locali_dplan_host_view(const void *const *src_host, int32_t n, uint64_t *out) {
    if (n < 0 || (n > 0 && (!src_host || !out))) return dfail(LOCALI_E_ARG, "dplan_host_view: bad arguments");
    for (int32_t i = 0; i < n; ++i) {
        void *dev = nullptr;
        if (!src_host[i] || reinterpret_cast<uintptr_t>(src_host[i]) % 16 ||
            hipHostGetDevicePointer(&dev, const_cast<void *>(src_host[i]), 0) != hipSuccess || dev != src_host[i]) {
            (void)hipGetLastError();
            return dfail(LOCALI_E_ARG, "dplan_host_view: source %d is not 16-byte aligned pinned host memory", i);
        }
        out[i] = reinterpret_cast<uint64_t>(dev);
    }
    return 0;
}

int locali_dplan_read(const void *state, locali_dplan_stats *stats, locali_cache_result *results,
                      int32_t max_results, void *stream) {
    if (!state || !stats || max_results < 0 || (max_results > 0 && !results))
        return dfail(LOCALI_E_ARG, "dplan_read: bad arguments");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    DPlanHeader h{};
    hipError_t e = hipMemcpyAsync(&h, state, sizeof(h), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return dhip(e, "dplan_read header");
    std::memset(stats, 0, sizeof(*stats));
    stats->hits = h.hits;
    stats->misses = h.misses;
    stats->evictions = h.evictions;
    stats->calls = h.calls;
    stats->error = h.error;
    stats->probation = h.count_probation;
    stats->protected_ = h.count_protected;
    stats->free_slots = h.free_count;
    stats->last_keys = h.n_want;
    stats->last_misses = h.n_miss;
    stats->prefetched = h.prefetched;
    stats->prefetch_used = h.pf_used;
    stats->prefetch_wasted = h.pf_wasted;
    if (max_results > 0 && h.n_want > 0) {
        const int32_t n = h.n_want < max_results ? h.n_want : max_results;
        const DPlanLayout G = dplan_layout(h.n_keys, h.n_slots, h.max_routes);
        e = hipMemcpyAsync(results, static_cast<const unsigned char *>(state) + G.res,
                           sizeof(locali_cache_result) * n, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return dhip(e, "dplan_read results");
    }
    return 0;
}

int32_t locali_dplan_peek(const void *state, int32_t key, void *stream) {
    if (!state || key < 0) return -1;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    DPlanHeader h{};
    if (hipMemcpyAsync(&h, state, sizeof(h), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess || key >= h.n_keys) {
        (void)hipGetLastError();
        return -1;
    }
    int32_t slot = -1;
    const DPlanLayout G = dplan_layout(h.n_keys, h.n_slots, h.max_routes);
    if (hipMemcpyAsync(&slot, static_cast<const unsigned char *>(state) + G.slot_of + sizeof(int32_t) * key,
                       sizeof(slot), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    return slot;
}

}  // extern "C"
