// C ABI of liblocali_amd.so (include/locali_moe.h): host-side validation,
// workspace carving and kernel launches. No allocation, no synchronisation.
#include "locali_moe.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "mfma_wide.hpp"
#include "launch.hpp"

using namespace locali;

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char *where) {
    return fail(LOCALI_E_HIP, "%s: %s", where, hipGetErrorString(e));
}

}  // namespace

namespace locali {
// The library's error record for entry points defined in other translation
// units (locali_moe_last_error reads it).
int set_error(int code, const char *msg) { return fail(code, "%s", msg); }
}  // namespace locali

namespace {

constexpr size_t kAlign = 256;
constexpr int kMaxSlots = 16000;
constexpr int kMaxExperts = 512;
constexpr int kRouterSplitsHost = 16;
constexpr int kDecodeMaxTokens = 2;   // above this the grouped path is used

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool dtype16(int32_t dt) { return dt == LOCALI_DT_F16 || dt == LOCALI_DT_BF16; }

// Workspace layout for up to T tokens.
struct Layout {
    size_t sync_gen, sync_logits, logits, route_slot, hidden, hprep, seg_start, seg_tile, sorted_route, route_pos,
        tiles, n_tiles, tile_tok, gh, gy, mx, mh, total;
    int max_tiles;
    int wide_tiles;   // tiles of the matrix-core path that tile_tok holds
};

// Bytes of one prepared vector of K values, for any bit width (pairs take at
// most K u32, partial sums at most K / 4 float2).
size_t prep_bytes(int K) { return align_up(4 * static_cast<size_t>(K)) + align_up(2 * static_cast<size_t>(K)); }

// Prepared inputs of the MFMA grouped kernels for n vectors of K values:
// pairs (K / 2 u32 each: at most 8 pairs per 16 values) then the per-64
// fixup operands (16 bytes each).
size_t mfma_batch_bytes(int n, int K) {
    return align_up(sizeof(uint32_t) * static_cast<size_t>(n) * (K / 2)) +
           align_up(sizeof(uint4) * static_cast<size_t>(n) * (K / 64 + 1));
}

MfmaVec mfma_batch(void *base, int n, int K) {
    MfmaVec v{};
    v.pairs = static_cast<uint32_t *>(base);
    v.pairs_stride = K / 2;
    v.fix = reinterpret_cast<uint4 *>(static_cast<char *>(base) +
                                      align_up(sizeof(uint32_t) * static_cast<size_t>(n) * (K / 2)));
    v.fix_stride = K / 64;
    return v;
}

Layout layout(int T, int d, int dff, int E, int k, int has_shared) {
    Layout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = align_up(off + bytes);
        return at;
    };
    const int R = T * k;
    const int routes = R + (has_shared ? T : 0);
    L.max_tiles = grouped_max_tiles(T, k, has_shared ? 1 : 0, E, kGroupedTileTokens);
    // The decode sync region sits at the same offsets for every call shape,
    // so calls of different sizes on one workspace agree on its generation.
    L.sync_gen = take(sizeof(uint32_t));
    L.sync_logits = take(sizeof(uint64_t) * kFusedRouterMaxTokens * kSyncMaxExperts);
    L.logits = take(sizeof(float) * kRouterSplitsHost * static_cast<size_t>(T) * E);
    L.route_slot = take(sizeof(int32_t) * R);
    L.hidden = take(sizeof(uint16_t) * static_cast<size_t>(routes) * dff);
    L.hprep = take(prep_bytes(dff) * routes);
    L.seg_start = take(sizeof(int32_t) * (kMaxSlots + 1));
    L.seg_tile = take(sizeof(int32_t) * kMaxSlots);
    L.sorted_route = take(sizeof(int32_t) * R);
    L.route_pos = take(sizeof(int32_t) * R);
    L.tiles = take(sizeof(int32_t) * 4 * L.max_tiles);
    L.n_tiles = take(sizeof(int32_t));
    // the matrix-core path's tiles of up to kWideTokens positions: their tokens
    L.wide_tiles = grouped_max_tiles(T, k, has_shared ? 1 : 0, E, kWideTokens);
    L.tile_tok = take(sizeof(int32_t) * kWideTokens * static_cast<size_t>(L.wide_tiles));
    L.gh = take(sizeof(uint16_t) * static_cast<size_t>(routes) * dff);
    L.gy = take(sizeof(uint16_t) * static_cast<size_t>(routes) * d);
    L.mx = take(mfma_batch_bytes(T, d));
    L.mh = take(mfma_batch_bytes(routes, dff));
    L.total = off;
    return L;
}

template <typename T>
T *at(void *ws, size_t off) {
    return reinterpret_cast<T *>(static_cast<char *>(ws) + off);
}

int check_proj(const locali_qproj &p, const char *name, int32_t x_dtype) {
    if (!p.weight || !p.scales || !p.biases)
        return fail(LOCALI_E_ARG, "%s: null array", name);
    if (p.bits != 2 && p.bits != 3 && p.bits != 4 && p.bits != 8)
        return fail(LOCALI_E_ARG, "%s: bits %d not in {2,3,4,8}", name, p.bits);
    if (p.group_size != 32 && p.group_size != 64 && p.group_size != 128)
        return fail(LOCALI_E_ARG, "%s: group_size %d not in {32,64,128}", name, p.group_size);
    if (p.rows <= 0 || p.cols <= 0 || p.cols % p.group_size)
        return fail(LOCALI_E_ARG, "%s: rows %d / cols %d invalid for group %d", name, p.rows, p.cols,
                    p.group_size);
    if (p.n_slots < 1) return fail(LOCALI_E_ARG, "%s: n_slots %d", name, p.n_slots);
    if (!dtype16(p.meta_dtype) || p.meta_dtype != x_dtype)
        return fail(LOCALI_E_ARG, "%s: metadata dtype %d must equal activation dtype %d", name,
                    p.meta_dtype, x_dtype);
    // chunk geometry in the width the kernels compute in (3-bit rows are
    // widened to 4-bit chunks of 32 values on load)
    const int lb = lane_bits(p.bits);
    const int64_t bits_row = static_cast<int64_t>(p.cols) * lb;
    const int64_t cpr = bits_row / 128;
    if (bits_row % 128 || !(cpr == 8 || cpr == 16 || cpr == 32 || cpr == 64 || cpr == 128 || cpr == 256))
        return fail(LOCALI_E_ARG,
                    "%s: cols*bits/128 = %lld 16-byte chunks per row unsupported "
                    "(need 8, 16, 32, 64, 128 or 256)",
                    name, static_cast<long long>(cpr));
    const int vpc = 128 / lb;
    if (p.group_size < vpc && !(p.bits == 2 && p.group_size == 32))
        return fail(LOCALI_E_ARG, "%s: group %d smaller than a 16-byte chunk", name, p.group_size);
    return 0;
}

QProj to_dev(const locali_qproj &p) {
    QProj q;
    q.w = static_cast<const uint32_t *>(p.weight);
    q.s = static_cast<const uint16_t *>(p.scales);
    q.b = static_cast<const uint16_t *>(p.biases);
    q.rows = p.rows;
    q.cols = p.cols;
    q.bits = p.bits;
    q.group = p.group_size;
    q.n_slots = p.n_slots;
    q.w_slot = static_cast<int64_t>(p.rows) * p.cols * p.bits / 32;
    q.m_slot = static_cast<int64_t>(p.rows) * p.cols / p.group_size;
    return q;
}

bool same_quant(const locali_qproj &a, const locali_qproj &b) {
    return a.bits == b.bits && a.group_size == b.group_size && a.rows == b.rows && a.cols == b.cols &&
           a.meta_dtype == b.meta_dtype;
}

int check_arena(const locali_expert_arena *a, const char *name, int32_t x_dtype, int d, int *dff) {
    if (!a) return fail(LOCALI_E_ARG, "%s: null arena", name);
    int rc;
    if ((rc = check_proj(a->gate, "gate", x_dtype)) || (rc = check_proj(a->up, "up", x_dtype)) ||
        (rc = check_proj(a->down, "down", x_dtype)))
        return rc;
    if (!same_quant(a->gate, a->up))
        return fail(LOCALI_E_ARG, "%s: gate and up projections must share shape and quantisation", name);
    if (a->gate.cols != d || a->down.rows != d || a->down.cols != a->gate.rows)
        return fail(LOCALI_E_ARG, "%s: shapes gate[%d,%d] down[%d,%d] inconsistent with d_model %d", name,
                    a->gate.rows, a->gate.cols, a->down.rows, a->down.cols, d);
    if (a->gate.n_slots != a->up.n_slots || a->gate.n_slots != a->down.n_slots)
        return fail(LOCALI_E_ARG, "%s: projections disagree on n_slots", name);
    *dff = a->gate.rows;
    return 0;
}

int check_shared(const locali_expert_arena *routed, const locali_expert_arena *shared) {
    if (!shared) return 0;
    if (!same_quant(routed->gate, shared->gate) || !same_quant(routed->up, shared->up) ||
        !same_quant(routed->down, shared->down))
        return fail(LOCALI_E_ARG, "shared expert must use the routed experts' shapes and quantisation");
    return 0;
}

hipStream_t S(void *stream) { return static_cast<hipStream_t>(stream); }

// n_vec prepared vectors of K values carved from `base` (see Layout).
PrepVec prep_view(void *base, int K, int bits, bool bf16) {
    PrepVec v{};
    v.pairs = static_cast<uint32_t *>(base);
    v.pairs_stride = prep_pairs_count(K, bits, bf16);
    v.parts_stride = prep_parts_count(K, bits);
    // all pairs first, then all parts: caller reserved prep_bytes(K) per vector
    return v;
}

PrepVec prep_batch(void *base, int n_vec, int K, int bits, bool bf16) {
    PrepVec v = prep_view(base, K, bits, bf16);
    const size_t pairs_bytes = align_up(4 * static_cast<size_t>(K) * n_vec);
    v.parts = reinterpret_cast<float2 *>(static_cast<char *>(base) + pairs_bytes);
    return v;
}

DecodeLaunch decode_launch(const locali_expert_arena *routed, const locali_expert_arena *shared, const void *x,
                           int32_t x_dtype, int32_t tokens, int32_t top_k, const int32_t *route_slot,
                           const float *weights, float limit, int32_t fp32_swiglu, int32_t combine_mode,
                           void *hidden, void *out, void *ws, const Layout &lay) {
    DecodeLaunch L{};
    L.ra.x = static_cast<const uint16_t *>(x);
    L.ra.route_slot = route_slot;
    L.ra.tokens = tokens;
    L.ra.top_k = top_k;
    L.ra.n_shared = shared ? 1 : 0;
    L.routes = tokens * top_k + (shared ? tokens : 0);
    L.bf16 = x_dtype == LOCALI_DT_BF16;
    L.gate = to_dev(routed->gate);
    L.up = to_dev(routed->up);
    L.down = to_dev(routed->down);
    const locali_expert_arena *sh = shared ? shared : routed;
    L.sgate = to_dev(sh->gate);
    L.sup = to_dev(sh->up);
    L.sdown = to_dev(sh->down);
    L.h = static_cast<uint16_t *>(hidden);
    L.limit = limit;
    L.fp32_swiglu = fp32_swiglu;
    L.ca.weights = weights;
    L.ca.out = static_cast<uint16_t *>(out);
    L.ca.mode = combine_mode;
    L.ca.gen = at<uint32_t>(ws, lay.sync_gen);
    const bool bf16 = x_dtype == LOCALI_DT_BF16;
    L.hprep = prep_batch(at<void>(ws, lay.hprep), L.routes, routed->down.cols, lane_bits(routed->down.bits),
                         bf16);
    return L;
}

// stages: bit 0 = gate/up, bit 1 = down + combine. sel: the gate/up kernel
// selects the routes itself (forward with a deferred selection).
int run_decode(const locali_expert_arena *routed, const locali_expert_arena *shared, const void *x,
               int32_t x_dtype, int32_t tokens, int32_t top_k, const int32_t *route_slot,
               const float *weights, float limit, int32_t fp32_swiglu, int32_t combine_mode,
               void *hidden, void *out, hipStream_t st, int stages, void *ws, const Layout &lay,
               const RouterLaunch *sel = nullptr) {
    DecodeLaunch L = decode_launch(routed, shared, x, x_dtype, tokens, top_k, route_slot, weights, limit,
                                   fp32_swiglu, combine_mode, hidden, out, ws, lay);
    L.sel = sel;
    hipError_t e;
    if ((stages & 1) && (e = launch_gateup_decode(L, st)) != hipSuccess)
        return hip_fail(e, "gate/up decode launch");
    if ((stages & 2) && (e = launch_down_combine_decode(L, st)) != hipSuccess)
        return hip_fail(e, "down/combine decode launch");
    return 0;
}

int check_decode_args(const locali_expert_arena *routed, const locali_expert_arena *shared,
                      int32_t x_dtype, int32_t tokens, int32_t top_k, const int32_t *route_slot,
                      int32_t combine_mode) {
    int rc, dff = 0;
    if (!dtype16(x_dtype) || tokens < 1 || top_k < 1 || !route_slot)
        return fail(LOCALI_E_ARG, "expert_decode: bad arguments");
    if (!routed) return fail(LOCALI_E_ARG, "expert_decode: null arena");
    if ((rc = check_arena(routed, "routed", x_dtype, routed->gate.cols, &dff))) return rc;
    if ((rc = check_shared(routed, shared))) return rc;
    if (top_k + (shared ? 1 : 0) > 16) return fail(LOCALI_E_ARG, "expert_decode: top_k + shared > 16");
    if (combine_mode != LOCALI_COMBINE_ROUNDED && combine_mode != LOCALI_COMBINE_FP32)
        return fail(LOCALI_E_ARG, "expert_decode: combine_mode %d", combine_mode);
    return 0;
}

// The matrix-core grouped path needs 2-, 3- or 4-bit codes (gate and up
// alike; 3-bit rows run on the 4-bit 64-position kernels, every tile size),
// groups of a multiple of 64 with a multiple of 8 per row and at most
// kWideMetaMaxGroups (96: K up to 6144 in groups of 64), rows in multiples
// of 128, columns in multiples of kMfmaColsAlign, its staged scales, biases
// and sums within the LDS of a workgroup, and prepared inputs (2 bytes per value) below 2 GiB so
// that its buffer offsets stay 31-bit; the shared expert must match the
// routed one (they share prepared inputs).
bool mfma_eligible(const locali_expert_arena *routed, const locali_expert_arena *shared, int64_t tokens,
                   int64_t routes) {
    if (2 * tokens * routed->gate.cols >= (int64_t{1} << 31) ||
        2 * routes * routed->down.cols >= (int64_t{1} << 31))
        return false;
    auto ok = [](const locali_qproj &p) {
        return (p.bits == 2 || p.bits == 3 || p.bits == 4) && p.group_size % 64 == 0 && p.rows % kWideRows == 0 &&
               p.cols % kMfmaColsAlign == 0 && (p.cols / p.group_size) % 8 == 0 &&
               p.cols / p.group_size <= kWideMetaMaxGroups;
    };
    if (!ok(routed->gate) || !ok(routed->up) || !ok(routed->down)) return false;
    if (wide_lds_bytes(routed->gate.cols, 2) > kWideMaxLds || wide_lds_bytes(routed->down.cols, 1) > kWideMaxLds)
        return false;
    if (routed->gate.bits != routed->up.bits) return false;
    if (shared && (shared->gate.bits != routed->gate.bits || shared->up.bits != routed->up.bits ||
                   shared->down.bits != routed->down.bits || !ok(shared->gate) || !ok(shared->up) ||
                   !ok(shared->down)))
        return false;
    return true;
}

// Small-tile kernels (mfma_small.hpp): groups of 64 or 128, K of both
// stages a multiple of 512 and at most 4096, rows multiples of 32.
// Positions of the small-tile kernels' tiles: gate/up 2; down 2, or 4 in
// calls of at least kSmallDown4Tokens tokens, where tiles of three and four
// positions are common under skewed routing (the four-position down kernel is
// faster than the 64-position one on those tiles and slower than the
// two-position one on the rest).
constexpr int kSmallGateUpTileHost = 2, kSmallDown4Tokens = 256;
bool small_tiles_eligible(const locali_expert_arena *routed) {
    auto ok = [](const locali_qproj &p) {
        return (p.bits == 2 || p.bits == 4) && (p.group_size == 64 || p.group_size == 128) &&
               (p.cols / p.group_size) % 8 == 0 && p.cols % 512 == 0 && p.cols <= 4096 && p.rows % 32 == 0;
    };
    return ok(routed->gate) && ok(routed->up) && ok(routed->down);
}

// Second stream of the grouped matrix-core path, one per host thread and
// device (the events are reused call after call, so calls from one thread
// stay ordered; threads never share a set). Created on the first grouped call
// that is not under stream capture; calls that must not allocate
// (set_no_alloc_call) and calls made before it exists under capture keep
// every kernel on the caller's stream. Default priority, non-blocking.
struct AuxStream {
    hipStream_t s = nullptr;
    hipEvent_t ev[4] = {};
    bool failed = false;
};
constexpr int kAuxMaxDevices = 64;
// Calls of fewer tokens keep one stream: their kernels are short and
// latency-bound, and the fork and joins cost more than the overlap gives.
constexpr int kAuxStreamTokens = 256;
thread_local AuxStream g_aux[kAuxMaxDevices];
thread_local bool g_no_alloc_call = false;

AuxStream *aux_stream(hipStream_t st) {
    if (g_no_alloc_call) return nullptr;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kAuxMaxDevices) return nullptr;
    AuxStream &a = g_aux[dev];
    if (a.s) return &a;
    if (a.failed) return nullptr;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
    hipStream_t s = nullptr;
    bool ok = hipStreamCreateWithFlags(&s, hipStreamNonBlocking) == hipSuccess;
    for (int i = 0; ok && i < 4; ++i) ok = hipEventCreateWithFlags(&a.ev[i], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        for (hipEvent_t &ev : a.ev)
            if (ev) (void)hipEventDestroy(ev), ev = nullptr;
        if (s) (void)hipStreamDestroy(s);
        (void)hipGetLastError();
        a.failed = true;
        return nullptr;
    }
    a.s = s;
    return &a;
}

}  // namespace

namespace locali {
void set_no_alloc_call(bool on) { g_no_alloc_call = on; }
}  // namespace locali

namespace {

int run_grouped_mfma(const locali_expert_arena *routed, const locali_expert_arena *shared,
                     const void *x, int32_t x_dtype, int32_t tokens, int32_t top_k, int32_t n_experts,
                     const int32_t *route_slot, const float *weights, float limit,
                     int32_t fp32_swiglu, int32_t combine_mode, void *out, void *ws,
                     const Layout &lay, hipStream_t st, uint16_t *h_plain) {
    const int R = tokens * top_k;
    const int n_slots = routed->gate.n_slots;
    const int routes = R + (shared ? tokens : 0);
    int32_t *route_pos = at<int32_t>(ws, lay.route_pos);
    int32_t *tiles = at<int32_t>(ws, lay.tiles);
    int32_t *n_tiles = at<int32_t>(ws, lay.n_tiles);
    uint16_t *gy = at<uint16_t>(ws, lay.gy);
    const int max_tiles = grouped_max_tiles(tokens, top_k, shared ? 1 : 0, n_experts, kWideTokens);
    if (max_tiles > lay.max_tiles || max_tiles > lay.wide_tiles)
        return fail(LOCALI_E_WORKSPACE, "grouped: tile list too small");
    // Tiles of one or two positions (gate/up; down: up to four in calls of
    // many tokens) go to the small-tile kernels when the shapes allow; the
    // 64-position kernels skip them. The dispatch packs the tokens of a tile of one or
    // two positions into its record, and writes every routed tile's tokens by
    // position for the 64-position kernels.
    const bool small = small_tiles_eligible(routed);
    int32_t *tile_tok = at<int32_t>(ws, lay.tile_tok);
    // the dispatch's count step; its placement step runs in one launch with
    // the preparation of x (launch_mfma stage 5)
    MfmaLaunch L{};
    hipError_t e = launch_dispatch_count(route_slot, R, n_slots, shared ? tokens : 0, kWideTokens,
                                         at<int32_t>(ws, lay.seg_start), at<int32_t>(ws, lay.sorted_route),
                                         route_pos, tiles, n_tiles, max_tiles, st, at<int32_t>(ws, lay.seg_tile),
                                         top_k, small, tile_tok, &L.place);
    if (e != hipSuccess) return hip_fail(e, "dispatch launch");
    L.ta.x = static_cast<const uint16_t *>(x);
    L.ta.tiles = tiles;
    L.ta.n_tiles = n_tiles;
    L.ta.sorted_route = at<int32_t>(ws, lay.sorted_route);
    L.ta.tile_tok = tile_tok;
    L.ta.R = R;
    L.ta.top_k = top_k;
    L.gate = to_dev(routed->gate);
    L.up = to_dev(routed->up);
    L.down = to_dev(routed->down);
    const locali_expert_arena *sh = shared ? shared : routed;
    L.sgate = to_dev(sh->gate);
    L.sup = to_dev(sh->up);
    L.sdown = to_dev(sh->down);
    L.xin = mfma_batch(at<void>(ws, lay.mx), tokens, routed->gate.cols);
    L.hmid = mfma_batch(at<void>(ws, lay.mh), routes, routed->down.cols);
    L.hmid.plain = h_plain;
    L.hsum32 = at<float2>(ws, lay.gh);   // the VALU path's h buffer is free here
    L.small_down_positions = tokens >= kSmallDown4Tokens ? 4 : 2;
    // the four-position small down kernel also takes tiles whose h the
    // 64-position gate/up kernel writes (three or four positions): that
    // kernel writes their sums
    if (small && L.small_down_positions > 2) L.hmid.sum32 = L.hsum32;
    L.y = gy;
    L.limit = limit;
    L.fp32_swiglu = fp32_swiglu;
    L.max_tiles = max_tiles;
    L.tokens = tokens;
    L.routes = routes;
    const bool bf16 = x_dtype == LOCALI_DT_BF16;
    L.ta.min_count = small ? kSmallGateUpTileHost + 1 : 0;
    L.min_count_down = small ? L.small_down_positions + 1 : 0;
    // 5: placement + preparation of x; 1, 3: gate/up (64-position, small
    // tiles); 2, 4: down
    AuxStream *ax = small && tokens >= kAuxStreamTokens ? aux_stream(st) : nullptr;
    if (!ax) {
        const int order[5] = {5, 1, 3, 2, 4};
        for (int which : order) {
            if ((which == 3 || which == 4) && !small) continue;
            if ((e = launch_mfma(which, bf16, L, st)) != hipSuccess) return hip_fail(e, "grouped MFMA launch");
        }
    } else {
        // the small-tile kernels on the second stream beside the 64-position
        // ones: gate/up pair after 5, down pair after both gate/ups (the
        // small down kernel also reads h of tiles the 64-position gate/up
        // kernel wrote), joined before the combine
        const hipStream_t sa = ax->s;
        if ((e = launch_mfma(5, bf16, L, st)) != hipSuccess) return hip_fail(e, "grouped MFMA launch");
        if ((e = hipEventRecord(ax->ev[0], st)) != hipSuccess || (e = hipStreamWaitEvent(sa, ax->ev[0], 0)) != hipSuccess)
            return hip_fail(e, "grouped fork");
        if ((e = launch_mfma(1, bf16, L, st)) != hipSuccess || (e = launch_mfma(3, bf16, L, sa)) != hipSuccess)
            return hip_fail(e, "grouped MFMA launch");
        if ((e = hipEventRecord(ax->ev[1], sa)) != hipSuccess || (e = hipStreamWaitEvent(st, ax->ev[1], 0)) != hipSuccess ||
            (e = hipEventRecord(ax->ev[2], st)) != hipSuccess || (e = hipStreamWaitEvent(sa, ax->ev[2], 0)) != hipSuccess)
            return hip_fail(e, "grouped join");
        if ((e = launch_mfma(2, bf16, L, st)) != hipSuccess || (e = launch_mfma(4, bf16, L, sa)) != hipSuccess)
            return hip_fail(e, "grouped MFMA launch");
        if ((e = hipEventRecord(ax->ev[3], sa)) != hipSuccess || (e = hipStreamWaitEvent(st, ax->ev[3], 0)) != hipSuccess)
            return hip_fail(e, "grouped join");
    }
    const int d = routed->down.rows;
    e = launch_combine(gy, route_pos, shared ? gy + static_cast<int64_t>(R) * d : nullptr, weights, tokens,
                       top_k, d, combine_mode, bf16, static_cast<uint16_t *>(out), st);
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return 0;
}

int run_grouped(const locali_expert_arena *routed, const locali_expert_arena *shared, const void *x,
                int32_t x_dtype, int32_t tokens, int32_t top_k, int32_t n_experts,
                const int32_t *route_slot, const float *weights, float limit, int32_t fp32_swiglu,
                int32_t combine_mode, void *out, void *ws, const Layout &lay, hipStream_t st,
                uint16_t *h_plain = nullptr, bool *on_mfma = nullptr) {
    const bool mfma =
        mfma_eligible(routed, shared, tokens, static_cast<int64_t>(tokens) * (top_k + (shared ? 1 : 0)));
    if (on_mfma) *on_mfma = mfma;
    if (mfma)
        return run_grouped_mfma(routed, shared, x, x_dtype, tokens, top_k, n_experts, route_slot, weights, limit,
                                fp32_swiglu, combine_mode, out, ws, lay, st, h_plain);
    const int R = tokens * top_k;
    const int n_slots = routed->gate.n_slots;
    int32_t *seg_start = at<int32_t>(ws, lay.seg_start);
    int32_t *sorted_route = at<int32_t>(ws, lay.sorted_route);
    int32_t *route_pos = at<int32_t>(ws, lay.route_pos);
    int32_t *tiles = at<int32_t>(ws, lay.tiles);
    int32_t *n_tiles = at<int32_t>(ws, lay.n_tiles);
    uint16_t *gh = at<uint16_t>(ws, lay.gh);
    uint16_t *gy = at<uint16_t>(ws, lay.gy);
    (void)n_experts;
    hipError_t e = launch_dispatch(route_slot, R, n_slots, shared ? tokens : 0, kGroupedTileTokens,
                                   seg_start, sorted_route, route_pos, tiles, n_tiles, lay.max_tiles, st);
    if (e != hipSuccess) return hip_fail(e, "dispatch launch");
    GroupedKernelLaunch G{};
    G.ta.x = static_cast<const uint16_t *>(x);
    G.ta.tiles = tiles;
    G.ta.n_tiles = n_tiles;
    G.ta.sorted_route = sorted_route;
    G.ta.R = R;
    G.ta.top_k = top_k;
    G.bf16 = x_dtype == LOCALI_DT_BF16;
    G.gate = to_dev(routed->gate);
    G.up = to_dev(routed->up);
    G.down = to_dev(routed->down);
    const locali_expert_arena *sh = shared ? shared : routed;
    G.sgate = to_dev(sh->gate);
    G.sup = to_dev(sh->up);
    G.sdown = to_dev(sh->down);
    G.h = gh;
    G.y = gy;
    G.limit = limit;
    G.fp32_swiglu = fp32_swiglu;
    G.max_tiles = lay.max_tiles;
    if ((e = launch_grouped_kernels(0, G, st)) != hipSuccess) return hip_fail(e, "grouped gate/up launch");
    if ((e = launch_grouped_kernels(1, G, st)) != hipSuccess) return hip_fail(e, "grouped down launch");
    const int d = routed->down.rows;
    e = launch_combine(gy, route_pos, shared ? gy + static_cast<int64_t>(R) * d : nullptr, weights, tokens,
                       top_k, d, combine_mode, x_dtype == LOCALI_DT_BF16, static_cast<uint16_t *>(out), st);
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return 0;
}

int check_router(const locali_router *r, int d) {
    if (!r || !r->weight) return fail(LOCALI_E_ARG, "router: null");
    if (r->n_experts < 1 || r->n_experts > kMaxExperts)
        return fail(LOCALI_E_ARG, "router: n_experts %d not in [1, %d]", r->n_experts, kMaxExperts);
    if (r->top_k < 1 || r->top_k > 16 || r->top_k > r->n_experts)
        return fail(LOCALI_E_ARG, "router: top_k %d invalid", r->top_k);
    if (r->weight_dtype != LOCALI_DT_F32 && !dtype16(r->weight_dtype))
        return fail(LOCALI_E_ARG, "router: weight dtype %d", r->weight_dtype);
    if (r->score_func < 0 || r->score_func > 2) return fail(LOCALI_E_ARG, "router: score_func %d", r->score_func);
    if (d % 8) return fail(LOCALI_E_ARG, "router: d_model %d not a multiple of 8", d);
    if (r->tid2eid && r->vocab < 1) return fail(LOCALI_E_ARG, "router: hash table without vocab");
    return 0;
}

// Builds the router launch; with logits_only (and a decode-sized call whose
// gate/up kernel selects on its own, router_select_fusable) only the logits
// kernel is launched and `*launch` carries what that kernel needs.
RouterLaunch router_launch(const locali_router *router, const void *x, int32_t x_dtype, int32_t tokens,
                           int32_t d_model, const int32_t *input_ids, const float *logits_in,
                           const int32_t *slot_of_expert, int32_t n_slots, int32_t *idx, float *weights,
                           int32_t *route_slot, float *logits) {
    RouterLaunch L{};
    L.x = static_cast<const uint16_t *>(x);
    L.x_bf16 = x_dtype == LOCALI_DT_BF16;
    L.gate_w = router->weight;
    L.gate_dtype = router->weight_dtype;
    L.bias = router->score_bias;
    L.tid2eid = router->tid2eid;
    L.input_ids = input_ids;
    L.vocab = router->vocab;
    L.tokens = tokens;
    L.d = d_model;
    L.E = router->n_experts;
    L.top_k = router->top_k;
    L.score_func = router->score_func;
    L.norm_topk = router->norm_topk;
    L.routed_scale = router->routed_scale;
    L.slot_of_expert = slot_of_expert;
    L.n_slots = n_slots;
    L.idx = idx;
    L.weights = weights;
    L.route_slot = route_slot;
    L.logits = logits;
    L.logits_in = logits_in;
    return L;
}

int route(const locali_router *router, const void *x, int32_t x_dtype, int32_t tokens, int32_t d_model,
          const int32_t *input_ids, const float *logits_in, const int32_t *slot_of_expert,
          int32_t n_slots, int32_t *idx, float *weights, int32_t *route_slot, void *workspace,
          const Layout &lay, hipStream_t st, bool logits_only = false, RouterLaunch *launch = nullptr) {
    if (router->tid2eid && !input_ids) return fail(LOCALI_E_ARG, "router: hash routing needs input_ids");
    if (route_slot && (!slot_of_expert || n_slots < 1))
        return fail(LOCALI_E_ARG, "router: route_slot needs slot_of_expert and n_slots");
    const RouterLaunch L = router_launch(router, x, x_dtype, tokens, d_model, input_ids, logits_in, slot_of_expert,
                                         n_slots, idx, weights, route_slot, at<float>(workspace, lay.logits));
    if (launch) *launch = L;
    if (logits_only && !router_select_fusable(L)) return fail(LOCALI_E_ARG, "router: selection cannot be deferred");
    hipError_t e = launch_router(L, st, logits_only);
    if (e != hipSuccess) return hip_fail(e, "router launch");
    return 0;
}

}  // namespace

extern "C" {

const char *locali_moe_last_error(void) { return g_error.c_str(); }

size_t locali_moe_workspace_bytes(int32_t tokens, int32_t d_model, int32_t d_ff, int32_t n_experts,
                                  int32_t top_k, int32_t has_shared) {
    if (tokens < 1 || d_model < 1 || d_ff < 1 || n_experts < 1 || top_k < 1) return 0;
    return layout(tokens, d_model, d_ff, n_experts, top_k, has_shared).total;
}

int locali_moe_router(const locali_router *router, const void *x, int32_t x_dtype, int32_t tokens,
                      int32_t d_model, const int32_t *input_ids, const float *logits_in,
                      const int32_t *slot_of_expert, int32_t n_slots, int32_t *idx, float *weights,
                      int32_t *route_slot, void *workspace, size_t workspace_bytes, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    int rc;
    if ((rc = check_router(router, d_model))) return rc;
    if (tokens < 1 || !x || !dtype16(x_dtype) || !idx || !weights || !workspace)
        return fail(LOCALI_E_ARG, "router: bad tokens/x/outputs/workspace");
    const Layout lay = layout(tokens, d_model, 1, router->n_experts, router->top_k, 0);
    if (workspace_bytes < lay.route_slot)
        return fail(LOCALI_E_WORKSPACE, "router: workspace %zu < %zu bytes", workspace_bytes, lay.route_slot);
    return route(router, x, x_dtype, tokens, d_model, input_ids, logits_in, slot_of_expert, n_slots, idx,
                 weights, route_slot, workspace, lay, S(stream));
}

int locali_moe_dispatch(const int32_t *route_slot, int32_t tokens, int32_t top_k, int32_t n_slots,
                        int32_t *sorted_route, int32_t *seg_start, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    if (!route_slot || !sorted_route || !seg_start || tokens < 1 || top_k < 1 || n_slots < 1 ||
        n_slots > kMaxSlots)
        return fail(LOCALI_E_ARG, "dispatch: bad arguments");
    // No tile list is produced for this entry point.
    hipError_t e = launch_dispatch(route_slot, tokens * top_k, n_slots, 0, 1, seg_start, sorted_route,
                                   nullptr, nullptr, nullptr, 0, S(stream));
    if (e != hipSuccess) return hip_fail(e, "dispatch launch");
    return 0;
}

int decode_workspace(const locali_expert_arena *routed, const locali_expert_arena *shared, int tokens,
                     int top_k, size_t workspace_bytes, void *workspace, Layout *lay) {
    if (!workspace) return fail(LOCALI_E_ARG, "decode: null workspace");
    *lay = layout(tokens, routed->gate.cols, routed->gate.rows, 1, top_k, shared ? 1 : 0);
    if (workspace_bytes < lay->total)
        return fail(LOCALI_E_WORKSPACE, "decode: workspace %zu < %zu bytes", workspace_bytes, lay->total);
    return 0;
}

int locali_moe_expert_decode(const locali_expert_arena *routed, const locali_expert_arena *shared,
                             const void *x, int32_t x_dtype, int32_t tokens, int32_t top_k,
                             const int32_t *route_slot, const float *weights, float swiglu_limit,
                             int32_t fp32_swiglu, int32_t combine_mode, void *hidden, void *out,
                             void *workspace, size_t workspace_bytes, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    if (!x || !weights || !hidden || !out) return fail(LOCALI_E_ARG, "expert_decode: null buffer");
    int rc = check_decode_args(routed, shared, x_dtype, tokens, top_k, route_slot, combine_mode);
    if (rc) return rc;
    Layout lay;
    if ((rc = decode_workspace(routed, shared, tokens, top_k, workspace_bytes, workspace, &lay))) return rc;
    return run_decode(routed, shared, x, x_dtype, tokens, top_k, route_slot, weights, swiglu_limit,
                      fp32_swiglu, combine_mode, hidden, out, S(stream), 3, workspace, lay);
}

int locali_moe_decode_gateup(const locali_expert_arena *routed, const locali_expert_arena *shared,
                             const void *x, int32_t x_dtype, int32_t tokens, int32_t top_k,
                             const int32_t *route_slot, float swiglu_limit, int32_t fp32_swiglu,
                             void *hidden, void *workspace, size_t workspace_bytes, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    if (!x || !hidden) return fail(LOCALI_E_ARG, "decode_gateup: null buffer");
    int rc = check_decode_args(routed, shared, x_dtype, tokens, top_k, route_slot,
                               LOCALI_COMBINE_ROUNDED);
    if (rc) return rc;
    Layout lay;
    if ((rc = decode_workspace(routed, shared, tokens, top_k, workspace_bytes, workspace, &lay))) return rc;
    return run_decode(routed, shared, x, x_dtype, tokens, top_k, route_slot, nullptr, swiglu_limit,
                      fp32_swiglu, LOCALI_COMBINE_ROUNDED, hidden, nullptr, S(stream), 1,
                      workspace, lay);
}

int locali_moe_decode_down_combine(const locali_expert_arena *routed,
                                   const locali_expert_arena *shared, int32_t x_dtype, int32_t tokens,
                                   int32_t top_k, const int32_t *route_slot, const float *weights,
                                   int32_t combine_mode, void *out, void *workspace,
                                   size_t workspace_bytes, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    if (!weights || !out) return fail(LOCALI_E_ARG, "decode_down_combine: null buffer");
    int rc = check_decode_args(routed, shared, x_dtype, tokens, top_k, route_slot, combine_mode);
    if (rc) return rc;
    Layout lay;
    if ((rc = decode_workspace(routed, shared, tokens, top_k, workspace_bytes, workspace, &lay))) return rc;
    return run_decode(routed, shared, nullptr, x_dtype, tokens, top_k, route_slot, weights, 0.f, 0,
                      combine_mode, at<void>(workspace, lay.hidden), out, S(stream), 2,
                      workspace, lay);
}

int locali_moe_expert_grouped(const locali_expert_arena *routed, const locali_expert_arena *shared,
                              const void *x, int32_t x_dtype, int32_t tokens, int32_t top_k,
                              int32_t n_experts, const int32_t *idx, const int32_t *slot_of_expert,
                              const float *weights, float swiglu_limit, int32_t fp32_swiglu,
                              int32_t combine_mode, void *out, void *workspace, size_t workspace_bytes,
                              void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    int rc, dff = 0;
    if (!x || !dtype16(x_dtype) || tokens < 1 || top_k < 1 || !idx || !slot_of_expert || !weights ||
        !out || !workspace || n_experts < 1)
        return fail(LOCALI_E_ARG, "expert_grouped: bad arguments");
    if (!routed) return fail(LOCALI_E_ARG, "expert_grouped: null arena");
    const int d = routed->gate.cols;
    if ((rc = check_arena(routed, "routed", x_dtype, d, &dff))) return rc;
    if ((rc = check_shared(routed, shared))) return rc;
    if (routed->gate.n_slots > kMaxSlots) return fail(LOCALI_E_ARG, "expert_grouped: n_slots > %d", kMaxSlots);
    const Layout lay = layout(tokens, d, dff, n_experts, top_k, shared ? 1 : 0);
    if (workspace_bytes < lay.total)
        return fail(LOCALI_E_WORKSPACE, "expert_grouped: workspace %zu < %zu bytes", workspace_bytes, lay.total);
    int32_t *route_slot = at<int32_t>(workspace, lay.route_slot);
    hipError_t e = launch_route_slots(idx, tokens * top_k, n_experts, slot_of_expert, routed->gate.n_slots,
                                      route_slot, S(stream));
    if (e != hipSuccess) return hip_fail(e, "route slot launch");
    return run_grouped(routed, shared, x, x_dtype, tokens, top_k, n_experts, route_slot, weights,
                       swiglu_limit, fp32_swiglu, combine_mode, out, workspace, lay, S(stream));
}

int locali_moe_expert_grouped_stages(const locali_expert_arena *routed, const locali_expert_arena *shared,
                                     const void *x, int32_t x_dtype, int32_t tokens, int32_t top_k,
                                     int32_t n_experts, const int32_t *idx, const int32_t *slot_of_expert,
                                     const float *weights, float swiglu_limit, int32_t fp32_swiglu,
                                     int32_t combine_mode, void *out, void *h_out, void *y_out,
                                     int32_t *route_pos_out, void *workspace, size_t workspace_bytes,
                                     void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    int rc, dff = 0;
    if (!x || !dtype16(x_dtype) || tokens < 1 || top_k < 1 || !idx || !slot_of_expert || !weights || !out ||
        !h_out || !y_out || !route_pos_out || !workspace || n_experts < 1 || !routed)
        return fail(LOCALI_E_ARG, "expert_grouped_stages: bad arguments");
    const int d = routed->gate.cols;
    if ((rc = check_arena(routed, "routed", x_dtype, d, &dff))) return rc;
    if ((rc = check_shared(routed, shared))) return rc;
    if (routed->gate.n_slots > kMaxSlots)
        return fail(LOCALI_E_ARG, "expert_grouped_stages: n_slots > %d", kMaxSlots);
    const Layout lay = layout(tokens, d, dff, n_experts, top_k, shared ? 1 : 0);
    if (workspace_bytes < lay.total)
        return fail(LOCALI_E_WORKSPACE, "expert_grouped_stages: workspace %zu < %zu bytes", workspace_bytes,
                    lay.total);
    const hipStream_t st = S(stream);
    int32_t *route_slot = at<int32_t>(workspace, lay.route_slot);
    hipError_t e = launch_route_slots(idx, tokens * top_k, n_experts, slot_of_expert, routed->gate.n_slots,
                                      route_slot, st);
    if (e != hipSuccess) return hip_fail(e, "route slot launch");
    bool mfma = false;
    if ((rc = run_grouped(routed, shared, x, x_dtype, tokens, top_k, n_experts, route_slot, weights, swiglu_limit,
                          fp32_swiglu, combine_mode, out, workspace, lay, st, static_cast<uint16_t *>(h_out),
                          &mfma)))
        return rc;
    const size_t R = static_cast<size_t>(tokens) * top_k, routes = R + (shared ? tokens : 0);
    if (!mfma &&   // the VALU kernels keep h by position in the workspace
        (e = hipMemcpyAsync(h_out, at<void>(workspace, lay.gh), routes * dff * sizeof(uint16_t),
                            hipMemcpyDeviceToDevice, st)) != hipSuccess)
        return hip_fail(e, "expert_grouped_stages h copy");
    if ((e = hipMemcpyAsync(y_out, at<void>(workspace, lay.gy), routes * d * sizeof(uint16_t),
                            hipMemcpyDeviceToDevice, st)) != hipSuccess ||
        (e = hipMemcpyAsync(route_pos_out, at<void>(workspace, lay.route_pos), R * sizeof(int32_t),
                            hipMemcpyDeviceToDevice, st)) != hipSuccess)
        return hip_fail(e, "expert_grouped_stages copies");
    return 0;
}

int locali_moe_combine(const void *y, const void *shared_y, const float *weights, int32_t dtype,
                       int32_t tokens, int32_t top_k, int32_t d, int32_t combine_mode, void *out,
                       void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    if (!y || !weights || !out || !dtype16(dtype) || tokens < 1 || top_k < 1 || d < 1)
        return fail(LOCALI_E_ARG, "combine: bad arguments");
    hipError_t e = launch_combine(static_cast<const uint16_t *>(y), nullptr,
                                  static_cast<const uint16_t *>(shared_y), weights, tokens, top_k, d,
                                  combine_mode, dtype == LOCALI_DT_BF16, static_cast<uint16_t *>(out),
                                  S(stream));
    if (e != hipSuccess) return hip_fail(e, "combine launch");
    return 0;
}

int locali_moe_combine_routes(const void *y, int32_t y_dtype, const int32_t *route_pos,
                              const void *shared_y, const float *weights, int32_t out_dtype,
                              int32_t tokens, int32_t top_k, int32_t d, int32_t combine_mode,
                              void *out, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    if (!y || !route_pos || !weights || !out || !dtype16(out_dtype) || tokens < 1 || top_k < 1 || d < 1)
        return fail(LOCALI_E_ARG, "combine_routes: bad arguments");
    if (y_dtype != LOCALI_DT_F32 && !dtype16(y_dtype))
        return fail(LOCALI_E_ARG, "combine_routes: y dtype %d", y_dtype);
    if (combine_mode != LOCALI_COMBINE_ROUNDED && combine_mode != LOCALI_COMBINE_FP32)
        return fail(LOCALI_E_ARG, "combine_routes: combine mode %d", combine_mode);
    const int y_type = y_dtype == LOCALI_DT_F32 ? 0 : (y_dtype == LOCALI_DT_F16 ? 1 : 2);
    hipError_t e = launch_combine_routes(y, y_type, route_pos, static_cast<const uint16_t *>(shared_y), weights,
                                         tokens, top_k, d, combine_mode, out_dtype == LOCALI_DT_BF16,
                                         static_cast<uint16_t *>(out), S(stream));
    if (e != hipSuccess) return hip_fail(e, "combine_routes launch");
    return 0;
}

int locali_moe_expert_prefill(const locali_expert_arena *routed, const locali_expert_arena *shared,
                              const void *x, int32_t x_dtype, int32_t tokens, int32_t top_k,
                              int32_t n_experts, const int32_t *idx, const int32_t *slot_of_expert,
                              const float *weights, float swiglu_limit, int32_t fp32_swiglu,
                              int32_t combine_mode, void *out, void *workspace, size_t workspace_bytes,
                              void *stream) {
    return locali_moe_expert_grouped(routed, shared, x, x_dtype, tokens, top_k, n_experts, idx, slot_of_expert,
                                     weights, swiglu_limit, fp32_swiglu, combine_mode, out, workspace,
                                     workspace_bytes, stream);
}

int locali_moe_arena_fill(void *dst, const void *src_host, size_t bytes, void *stream) {
    if (!dst || !src_host) return fail(LOCALI_E_ARG, "arena_fill: null pointer");
    if (!bytes) return 0;
    hipError_t e = hipMemcpyAsync(dst, src_host, bytes, hipMemcpyHostToDevice, S(stream));
    if (e != hipSuccess) return hip_fail(e, "arena_fill");
    return 0;
}

}  // extern "C"

namespace {

// Pieces for the fill kernel, launched 64 pieces at a time.
struct FillQueue {
    FillBatch b{};
    int blocks = 0;
    hipStream_t st;
    const char *what;
    explicit FillQueue(hipStream_t s, const char *w) : st(s), what(w) {}
    int flush() {
        if (!b.n) return 0;
        const hipError_t e = launch_fill(b, blocks, st);
        b.n = 0;
        blocks = 0;
        return e != hipSuccess ? hip_fail(e, what) : 0;
    }
    // dev_src: the device's address of pinned host memory at src (the same
    // address under unified addressing), or null: then an asynchronous copy
    int add(void *dst, const void *src, const void *dev_src, size_t bytes) {
        if (!bytes) return 0;
        if (!dev_src || (reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) | bytes) % 16) {
            const hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st);
            return e != hipSuccess ? hip_fail(e, what) : 0;
        }
        const int64_t units = static_cast<int64_t>(bytes / 16);
        const int nb = fill_blocks(units);
        if (b.n == kFillMaxPieces || static_cast<int64_t>(blocks) + nb > (int64_t{1} << 30)) {
            if (int rc = flush()) return rc;
        }
        b.first_block[b.n] = blocks;
        b.units[b.n] = units;
        b.src[b.n] = dev_src;
        b.dst[b.n] = dst;
        ++b.n;
        blocks += nb;
        return 0;
    }
};

// The kernel reads only pinned memory that the runtime maps at the same
// address on the device; anything else is copied.
const void *device_view(const void *host) {
    void *dev = nullptr;
    if (hipHostGetDevicePointer(&dev, const_cast<void *>(host), 0) != hipSuccess || dev != host) {
        (void)hipGetLastError();   // not pinned here
        return nullptr;
    }
    return dev;
}

}  // namespace

extern "C" {

int locali_moe_arena_fill_batch(const locali_fill_piece *pieces, int32_t n, void *stream) {
    if (n < 0 || (n > 0 && !pieces)) return fail(LOCALI_E_ARG, "arena_fill_batch: bad piece table");
    FillQueue q(S(stream), "arena_fill_batch");
    for (int32_t i = 0; i < n; ++i) {
        const locali_fill_piece &p = pieces[i];
        if (!p.bytes) continue;
        if (!p.dst || !p.src_host) return fail(LOCALI_E_ARG, "arena_fill_batch: null pointer in piece %d", i);
        if (int rc = q.add(p.dst, p.src_host, device_view(p.src_host), p.bytes)) return rc;
    }
    return q.flush();
}

int locali_moe_arena_fill_slots(void *const *dst_base, const size_t *slot_bytes, int32_t n_arrays,
                                int32_t n_slots, const int32_t *slots, const void *const *src_host, int32_t n,
                                void *stream) {
    if (n < 0 || n_arrays < 1 || n_slots < 1 || (n > 0 && (!dst_base || !slot_bytes || !slots || !src_host)))
        return fail(LOCALI_E_ARG, "arena_fill_slots: bad arguments");
    for (int32_t a = 0; a < n_arrays; ++a)
        if (!dst_base[a]) return fail(LOCALI_E_ARG, "arena_fill_slots: null array %d", a);
    // every argument is checked before the first copy is queued
    for (int32_t i = 0; i < n; ++i) {
        if (!src_host[i]) return fail(LOCALI_E_ARG, "arena_fill_slots: null source %d", i);
        if (slots[i] < 0 || slots[i] >= n_slots)
            return fail(LOCALI_E_ARG, "arena_fill_slots: slot %d of expert %d outside [0, %d)", slots[i], i, n_slots);
    }
    FillQueue q(S(stream), "arena_fill_slots");
    for (int32_t i = 0; i < n; ++i) {
        const char *src = static_cast<const char *>(src_host[i]);
        const char *dev = static_cast<const char *>(device_view(src));
        size_t off = 0;
        for (int32_t a = 0; a < n_arrays; ++a) {
            char *dst = static_cast<char *>(dst_base[a]) + static_cast<size_t>(slots[i]) * slot_bytes[a];
            if (int rc = q.add(dst, src + off, dev ? dev + off : nullptr, slot_bytes[a])) return rc;
            off += slot_bytes[a];
        }
    }
    return q.flush();
}

int locali_moe_router_logits(const locali_router *router, const void *x, int32_t x_dtype, int32_t tokens,
                             int32_t d_model, float *logits, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    int rc;
    if ((rc = check_router(router, d_model))) return rc;
    if (!x || !logits || tokens < 1 || !dtype16(x_dtype)) return fail(LOCALI_E_ARG, "router_logits: bad arguments");
    if (tokens > kFusedSelectMaxTokens)
        return fail(LOCALI_E_ARG, "router_logits: %d tokens; at most %d (decode)", tokens, kFusedSelectMaxTokens);
    const RouterLaunch L = router_launch(router, x, x_dtype, tokens, d_model, nullptr, nullptr, nullptr, 0, nullptr,
                                         nullptr, nullptr, logits);
    hipError_t e = launch_router(L, S(stream), true);
    if (e != hipSuccess) return hip_fail(e, "router_logits launch");
    return 0;
}

int locali_moe_decode_gateup_select(const locali_router *router, const locali_expert_arena *routed,
                                    const locali_expert_arena *shared, const int32_t *slot_of_expert,
                                    const void *x, int32_t x_dtype, int32_t tokens, const int32_t *input_ids,
                                    const float *logits, float swiglu_limit, int32_t fp32_swiglu, int32_t *idx,
                                    float *weights, int32_t *route_slot, void *hidden, void *workspace,
                                    size_t workspace_bytes, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    int rc, dff = 0;
    if (!routed || !x || !logits || !idx || !weights || !route_slot || !hidden || !workspace || !slot_of_expert ||
        tokens < 1 || !dtype16(x_dtype))
        return fail(LOCALI_E_ARG, "decode_gateup_select: bad arguments");
    const int d = routed->gate.cols;
    if ((rc = check_router(router, d))) return rc;
    if ((rc = check_arena(routed, "routed", x_dtype, d, &dff))) return rc;
    if ((rc = check_shared(routed, shared))) return rc;
    if (router->tid2eid && !input_ids) return fail(LOCALI_E_ARG, "decode_gateup_select: hash routing needs input_ids");
    const int k = router->top_k;
    if (tokens > kDecodeMaxTokens)
        return fail(LOCALI_E_ARG, "decode_gateup_select: %d tokens; at most %d", tokens, kDecodeMaxTokens);
    if (k + (shared ? 1 : 0) > 16) return fail(LOCALI_E_ARG, "decode_gateup_select: top_k + shared > 16");
    if (routed->gate.n_slots > kMaxSlots) return fail(LOCALI_E_ARG, "decode_gateup_select: n_slots > %d", kMaxSlots);
    // the decode stages' layout (no logits region: the logits are the caller's), so
    // that locali_moe_decode_down_combine finds the prepared hidden vectors
    const Layout lay = layout(tokens, d, dff, 1, k, shared ? 1 : 0);
    if (workspace_bytes < lay.total)
        return fail(LOCALI_E_WORKSPACE, "decode_gateup_select: workspace %zu < %zu bytes", workspace_bytes, lay.total);
    const RouterLaunch RL = router_launch(router, x, x_dtype, tokens, d, input_ids, nullptr, slot_of_expert,
                                          routed->gate.n_slots, idx, weights, route_slot, const_cast<float *>(logits));
    const DecodeLaunch DL = decode_launch(routed, shared, x, x_dtype, tokens, k, route_slot, weights, swiglu_limit,
                                          fp32_swiglu, LOCALI_COMBINE_ROUNDED, hidden, nullptr, workspace, lay);
    if (!router_select_fusable(RL) || !gateup_diag_eligible(DL))
        return fail(LOCALI_E_ARG, "decode_gateup_select: needs n_experts <= 256, a gate/up of 2-, 3- or 4-bit "
                                  "codes in groups of 64 or 128 with d_model a multiple of 512 up to 4096 and "
                                  "d_ff a multiple of 32, and a down projection of 2, 3 or 4 bits");
    return run_decode(routed, shared, x, x_dtype, tokens, k, route_slot, weights, swiglu_limit, fp32_swiglu,
                      LOCALI_COMBINE_ROUNDED, hidden, nullptr, S(stream), 1, workspace, lay, &RL);
}

int locali_moe_forward(const locali_router *router, const locali_expert_arena *routed,
                       const locali_expert_arena *shared, const int32_t *slot_of_expert, const void *x,
                       int32_t x_dtype, int32_t tokens, const int32_t *input_ids, float swiglu_limit,
                       int32_t fp32_swiglu, void *out, int32_t *idx, float *weights, void *workspace,
                       size_t workspace_bytes, void *stream) {
    if (tokens == 0) return 0;   // an empty batch is a no-op
    int rc, dff = 0;
    if (!routed || !x || !out || !idx || !weights || !workspace || !slot_of_expert || tokens < 1 ||
        !dtype16(x_dtype))
        return fail(LOCALI_E_ARG, "forward: bad arguments");
    const int d = routed->gate.cols;
    if ((rc = check_router(router, d))) return rc;
    if ((rc = check_arena(routed, "routed", x_dtype, d, &dff))) return rc;
    if ((rc = check_shared(routed, shared))) return rc;
    const int k = router->top_k, E = router->n_experts;
    if (k + (shared ? 1 : 0) > 16) return fail(LOCALI_E_ARG, "forward: top_k + shared > 16");
    if (routed->gate.n_slots > kMaxSlots) return fail(LOCALI_E_ARG, "forward: n_slots > %d", kMaxSlots);
    const Layout lay = layout(tokens, d, dff, E, k, shared ? 1 : 0);
    if (workspace_bytes < lay.total)
        return fail(LOCALI_E_WORKSPACE, "forward: workspace %zu < %zu bytes", workspace_bytes, lay.total);
    int32_t *route_slot = at<int32_t>(workspace, lay.route_slot);
    const bool decode = tokens <= kDecodeMaxTokens;
    // Decode: the gate/up kernel selects each token's routes itself when it
    // can, which saves the select kernel between the logits and the experts.
    bool defer = false;
    if (decode) {
        RouterLaunch probe{};
        probe.tokens = tokens;
        probe.E = E;
        probe.top_k = k;
        const DecodeLaunch DL = decode_launch(routed, shared, x, x_dtype, tokens, k, route_slot, weights,
                                              swiglu_limit, fp32_swiglu, LOCALI_COMBINE_ROUNDED,
                                              at<void>(workspace, lay.hidden), out, workspace, lay);
        defer = router_select_fusable(probe) && gateup_diag_eligible(DL);
    }
    RouterLaunch RL{};
    if (defer) {
        // The gate/up kernel also computes the logits (router rows ahead of
        // its gate/up rows) when the router allows it: no logits kernel.
        RL = router_launch(router, x, x_dtype, tokens, d, input_ids, nullptr, slot_of_expert, routed->gate.n_slots,
                           idx, weights, route_slot, at<float>(workspace, lay.logits));
        if (router->tid2eid && !input_ids) return fail(LOCALI_E_ARG, "router: hash routing needs input_ids");
        if (router_rows_fusable(RL)) {
            // Router work goes to the shared expert's rows (first in the grid,
            // waiting for nothing), up to 4 experts per workgroup; rows of
            // router work only make up any shortfall.
            const int tiles = dff / (16 * kDiagGateUpTiles), waves = d / kDiagWindow;
            const int sh_rows = shared ? tokens : 0;
            int epw = waves < 2 ? waves : 2;
            if (sh_rows) epw = std::min(waves, std::max(1, (E + sh_rows * tiles - 1) / (sh_rows * tiles)));
            const int rest = std::max(0, E - sh_rows * tiles * epw);
            RL.sync_gen = at<uint32_t>(workspace, lay.sync_gen);
            RL.sync_logits = at<uint64_t>(workspace, lay.sync_logits);
            RL.router_epw = epw;
            RL.router_shared_rows = sh_rows;
            RL.router_rows = sh_rows + (rest + tiles * epw - 1) / (tiles * epw);
            return run_decode(routed, shared, x, x_dtype, tokens, k, route_slot, weights, swiglu_limit, fp32_swiglu,
                              LOCALI_COMBINE_ROUNDED, at<void>(workspace, lay.hidden), out, S(stream), 3,
                              workspace, lay, &RL);
        }
    }
    rc = route(router, x, x_dtype, tokens, d, input_ids, nullptr, slot_of_expert, routed->gate.n_slots,
               idx, weights, route_slot, workspace, lay, S(stream), defer, &RL);
    if (rc) return rc;
    if (decode)
        return run_decode(routed, shared, x, x_dtype, tokens, k, route_slot, weights, swiglu_limit,
                          fp32_swiglu, LOCALI_COMBINE_ROUNDED, at<void>(workspace, lay.hidden), out,
                          S(stream), 3, workspace, lay, defer ? &RL : nullptr);
    return run_grouped(routed, shared, x, x_dtype, tokens, k, E, route_slot, weights, swiglu_limit,
                       fp32_swiglu, LOCALI_COMBINE_ROUNDED, out, workspace, lay, S(stream));
}

}  // extern "C"
