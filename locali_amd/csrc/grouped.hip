// Grouped expert path (prefill and batched decode): dispatch, tile list and
// combine. The (token, k) route entries are sorted by arena slot, stably
// (token order inside a slot) as the reference mixed-tier path does
// (arena.py:641-659), so each slot's weights are streamed once per group of
// tokens instead of once per route.
//
//   dispatch_count_kernel   one workgroup: per-slot counts, exclusive scan
//                           (seg_start), per-slot tile counts and the tile
//                           list (slot, first position, token count); the
//                           shared expert, when present, is one more segment
//                           holding every token, whose tiles come first in the
//                           list (the longest tiles start with the launch);
//                           routes outside the arena get route_pos -1
//   dispatch_place_kernel   (dispatch_place_block; the matrix-core path runs it
//                           in one launch with the preparation of x)
//                           one wave per slot: walks the routes 512 at a time
//                           with ballots and writes sorted_route / route_pos
//                           in route order (stable), and on request each
//                           routed tile's tokens by position (tile_tok), so
//                           that a tile kernel reads them beside the tile's
//                           record instead of after it
//   combine_kernel          out[t] = round(sum_j round(y[pos(t,j)] * w)) (+ shared)
#include "mfma_grouped.hpp"

namespace locali {

constexpr int kDispatchThreads = 1024;
constexpr int kMaxDispatchSlots = 16000;   // counts live in 64 KiB of LDS

__global__ __launch_bounds__(kDispatchThreads) void dispatch_count_kernel(
    const int32_t *__restrict__ route_slot, int R, int n_slots, int n_shared_tokens, int tile_tokens,
    int32_t *__restrict__ seg_start, int32_t *__restrict__ tiles, int32_t *__restrict__ n_tiles,
    int max_tiles, int32_t *__restrict__ route_pos, int32_t *__restrict__ seg_tile, int small_pack) {
    // the shared expert's tiles first, then the routed segments in slot order
    const int n_shared_tiles = (n_shared_tokens + tile_tokens - 1) / tile_tokens;
    extern __shared__ int32_t cnt[];              // [n_slots + 1]
    __shared__ int32_t wsum[kDispatchThreads / 64];
    __shared__ int32_t carry;
    const int tid = threadIdx.x;
    for (int s = tid; s <= n_slots; s += blockDim.x) cnt[s] = 0;
    __syncthreads();
    for (int r = tid; r < R; r += blockDim.x) {
        const int s = route_slot[r];
        if (s >= 0 && s < n_slots) atomicAdd(&cnt[s], 1);
        else if (route_pos) route_pos[r] = -1;   // outside the arena: never placed
    }
    __syncthreads();
    // Two exclusive scans over slots in chunks of blockDim.x: positions and tiles.
    for (int pass = 0; pass < 2; ++pass) {
        if (tid == 0) carry = 0;
        __syncthreads();
        for (int base = 0; base < n_slots; base += blockDim.x) {
            const int s = base + tid;
            const int c = s < n_slots ? cnt[s] : 0;
            const int v = pass == 0 ? c : (c + tile_tokens - 1) / tile_tokens;
            // inclusive wave scan
            int x = v;
            for (int m = 1; m < 64; m <<= 1) {
                const int y = __shfl_up(x, m, 64);
                if ((tid & 63) >= m) x += y;
            }
            if ((tid & 63) == 63) wsum[tid >> 6] = x;
            __syncthreads();
            if (tid < 64) {
                int w = tid < (int)(blockDim.x >> 6) ? wsum[tid] : 0;
                for (int m = 1; m < 64; m <<= 1) {
                    const int y = __shfl_up(w, m, 64);
                    if (tid >= m) w += y;
                }
                if (tid < (int)(blockDim.x >> 6)) wsum[tid] = w;
            }
            __syncthreads();
            const int excl = carry + (tid >= 64 ? wsum[(tid >> 6) - 1] : 0) + x - v;
            if (s < n_slots) {
                if (pass == 0) {
                    seg_start[s] = excl;
                } else {
                    int pos = seg_start[s];
                    if (seg_tile) seg_tile[s] = n_shared_tiles + excl;
                    for (int q = 0; q < v; ++q) {
                        const int tile = n_shared_tiles + excl + q;
                        if (tiles && tile < max_tiles) {
                            const int first = pos + q * tile_tokens;
                            tiles[4 * tile + 0] = s;
                            tiles[4 * tile + 1] = first;
                            tiles[4 * tile + 2] = min(tile_tokens, c - q * tile_tokens);
                            // a tile of at most kPackedTokens positions gets its
                            // tokens from the place kernel (kTokensPacked marks it)
                            tiles[4 * tile + 3] = small_pack && c <= kPackedTokens ? kTokensPacked : 0;
                        }
                    }
                }
            }
            __syncthreads();
            if (tid == blockDim.x - 1) carry = excl + v;
            __syncthreads();
        }
        if (pass == 0 && tid == 0) seg_start[n_slots] = carry;
        __syncthreads();
    }
    if (tid == 0) {
        // shared expert: positions R .. R + n_shared_tokens, slot marker -2
        for (int q = 0; q < n_shared_tiles; ++q) {
            if (tiles && q < max_tiles) {
                tiles[4 * q + 0] = -2;
                tiles[4 * q + 1] = R + q * tile_tokens;
                tiles[4 * q + 2] = min(tile_tokens, n_shared_tokens - q * tile_tokens);
                tiles[4 * q + 3] = 0;
            }
        }
        if (n_tiles) *n_tiles = min(n_shared_tiles + carry, max_tiles);
    }
}

__global__ __launch_bounds__(256) void dispatch_place_kernel(PlaceArgs a) {
    dispatch_place_block(a, static_cast<int>(blockIdx.x));
}

// expert id -> slot, fused with the route list.
__global__ void route_slots_kernel(const int32_t *__restrict__ idx, int R, int E,
                                   const int32_t *__restrict__ slot_of_expert, int n_slots,
                                   int32_t *__restrict__ route_slot) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < R) {
        const int e = idx[r];
        int s = (e >= 0 && e < E) ? slot_of_expert[e] : -1;
        if (s >= n_slots) s = -1;
        route_slot[r] = s;
    }
}

template <bool BF16>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t *__restrict__ y,
                                                      const int32_t *__restrict__ route_pos,
                                                      const uint16_t *__restrict__ shared_y,
                                                      const float *__restrict__ weights, int tokens,
                                                      int top_k, int d, int mode,
                                                      uint16_t *__restrict__ out) {
    const int t = blockIdx.y;
    const int col = blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= d) return;
    float acc = 0.f;
    for (int j = 0; j < top_k; ++j) {
        const int r = t * top_k + j;
        const int p = route_pos ? route_pos[r] : r;
        if (p < 0) continue;
        const float w = round16<BF16>(weights[r]);
        const float v = to_float<BF16>(y[static_cast<int64_t>(p) * d + col]);
        acc += mode == 0 ? round16<BF16>(v * w) : v * w;
    }
    float o = round16<BF16>(acc);
    if (shared_y) o = round16<BF16>(o + to_float<BF16>(shared_y[static_cast<int64_t>(t) * d + col]));
    out[static_cast<int64_t>(t) * d + col] = from_float<BF16>(o);
}

// The same combine, eight consecutive columns per thread with 16-byte loads
// and stores (d a multiple of 8, rows 16-byte aligned); every element's
// arithmetic and order are those of combine_kernel.
template <bool BF16>
__global__ __launch_bounds__(256) void combine8_kernel(const uint16_t *__restrict__ y,
                                                       const int32_t *__restrict__ route_pos,
                                                       const uint16_t *__restrict__ shared_y,
                                                       const float *__restrict__ weights, int tokens,
                                                       int top_k, int d, int mode,
                                                       uint16_t *__restrict__ out) {
    const int t = blockIdx.y;
    const int c8 = blockIdx.x * blockDim.x + threadIdx.x;
    if (8 * c8 >= d) return;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
    for (int j = 0; j < top_k; ++j) {
        const int r = t * top_k + j;
        const int p = route_pos ? route_pos[r] : r;
        if (p < 0) continue;
        const float w = round16<BF16>(weights[r]);
        const uint4 v = reinterpret_cast<const uint4 *>(y + static_cast<int64_t>(p) * d)[c8];
        const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float f = to_float<BF16>(static_cast<uint16_t>(vw[i / 2] >> (16 * (i % 2))));
            acc[i] += mode == 0 ? round16<BF16>(f * w) : f * w;
        }
    }
    uint4 sv = make_uint4(0u, 0u, 0u, 0u);
    if (shared_y) sv = reinterpret_cast<const uint4 *>(shared_y + static_cast<int64_t>(t) * d)[c8];
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
    uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float v = round16<BF16>(acc[i]);
        if (shared_y) v = round16<BF16>(v + to_float<BF16>(static_cast<uint16_t>(sw[i / 2] >> (16 * (i % 2)))));
        o[i / 2] |= static_cast<uint32_t>(from_float<BF16>(v)) << (16 * (i % 2));
    }
    reinterpret_cast<uint4 *>(out + static_cast<int64_t>(t) * d)[c8] = make_uint4(o[0], o[1], o[2], o[3]);
}

// Weighted combine of route outputs held anywhere in `y`: route (t, j) reads
// row route_pos[t * top_k + j] (skipped when negative), in j order. YT is the
// rows' type (0 fp32, 1 fp16, 2 bf16); BF16 the output / shared / weight
// rounding type.
template <int YT>
__device__ __forceinline__ float load_row_value(const void *y, int64_t i) {
    if constexpr (YT == 0) return static_cast<const float *>(y)[i];
    else return to_float<YT == 2>(static_cast<const uint16_t *>(y)[i]);
}

template <int YT, bool BF16>
__global__ __launch_bounds__(256) void combine_routes_kernel(const void *__restrict__ y,
                                                             const int32_t *__restrict__ route_pos,
                                                             const uint16_t *__restrict__ shared_y,
                                                             const float *__restrict__ weights,
                                                             int top_k, int d, int mode,
                                                             uint16_t *__restrict__ out) {
    const int t = blockIdx.y;
    const int col = blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= d) return;
    float acc = 0.f;
    for (int j = 0; j < top_k; ++j) {
        const int r = t * top_k + j;
        const int p = route_pos[r];
        if (p < 0) continue;
        const float w = round16<BF16>(weights[r]);
        const float v = load_row_value<YT>(y, static_cast<int64_t>(p) * d + col);
        acc += mode == 0 ? round16<BF16>(v * w) : v * w;
    }
    float o = round16<BF16>(acc);
    if (shared_y) o = round16<BF16>(o + to_float<BF16>(shared_y[static_cast<int64_t>(t) * d + col]));
    out[static_cast<int64_t>(t) * d + col] = from_float<BF16>(o);
}

// --------------------------------------------------------------------------
hipError_t grouped_b2_bf16(int, int, int, const GroupedKernelLaunch &, hipStream_t);
hipError_t grouped_b2_f16(int, int, int, const GroupedKernelLaunch &, hipStream_t);
hipError_t grouped_b4_bf16(int, int, int, const GroupedKernelLaunch &, hipStream_t);
hipError_t grouped_b4_f16(int, int, int, const GroupedKernelLaunch &, hipStream_t);
hipError_t grouped_b8_bf16(int, int, int, const GroupedKernelLaunch &, hipStream_t);
hipError_t grouped_b8_f16(int, int, int, const GroupedKernelLaunch &, hipStream_t);
hipError_t grouped_b3_bf16(int, int, int, const GroupedKernelLaunch &, hipStream_t);
hipError_t grouped_b3_f16(int, int, int, const GroupedKernelLaunch &, hipStream_t);

// which: 0 = gate/up + SwiGLU, 1 = down.
hipError_t launch_grouped_kernels(int which, const GroupedKernelLaunch &L, hipStream_t st) {
    const QProj &p = which == 0 ? L.gate : L.down;
    const int gpc = group_parts(p), cpr = chunks_per_row(p);
    switch (p.bits) {
    case 2: return L.bf16 ? grouped_b2_bf16(which, gpc, cpr, L, st) : grouped_b2_f16(which, gpc, cpr, L, st);
    case 4: return L.bf16 ? grouped_b4_bf16(which, gpc, cpr, L, st) : grouped_b4_f16(which, gpc, cpr, L, st);
    case 8: return L.bf16 ? grouped_b8_bf16(which, gpc, cpr, L, st) : grouped_b8_f16(which, gpc, cpr, L, st);
    case 3: return L.bf16 ? grouped_b3_bf16(which, gpc, cpr, L, st) : grouped_b3_f16(which, gpc, cpr, L, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t mfma_b2(int which, bool bf16, const MfmaLaunch &L, hipStream_t st);
hipError_t mfma_b3(int which, bool bf16, const MfmaLaunch &L, hipStream_t st);
hipError_t mfma_b4(int which, bool bf16, const MfmaLaunch &L, hipStream_t st);

// which: 0 = prepare x, 1 = gate/up + SwiGLU (+ prepared h), 2 = down,
// 3 / 4 = gate/up / down of the small tiles, 5 = the dispatch's placement
// step (L.place) and the preparation of x in one launch. Gate and up share
// the prepared x, so they must share a bit width.
hipError_t launch_mfma(int which, bool bf16, const MfmaLaunch &L, hipStream_t st) {
    const int bits = which == 2 || which == 4 ? L.down.bits : L.gate.bits;
    switch (bits) {
    case 2: return mfma_b2(which, bf16, L, st);
    case 3: return mfma_b3(which, bf16, L, st);
    case 4: return mfma_b4(which, bf16, L, st);
    default: return hipErrorInvalidValue;
    }
}

int grouped_max_tiles(int tokens, int top_k, int n_shared, int E, int tile_tokens) {
    const int R = tokens * top_k;
    const int distinct = R < E ? R : E;
    return (R + tile_tokens - 1) / tile_tokens + distinct +
           n_shared * ((tokens + tile_tokens - 1) / tile_tokens) + 1;
}

hipError_t launch_dispatch_count(const int32_t *route_slot, int R, int n_slots, int n_shared_tokens,
                                 int tile_tokens, int32_t *seg_start, int32_t *sorted_route,
                                 int32_t *route_pos, int32_t *tiles, int32_t *n_tiles, int max_tiles,
                                 hipStream_t st, int32_t *seg_tile, int top_k, bool pack_small,
                                 int32_t *tile_tok, PlaceArgs *place) {
    if (n_slots < 1 || n_slots > kMaxDispatchSlots) return hipErrorInvalidValue;
    // tokens fit the packed field (and the tiles exist to hold it)
    const int pack = pack_small && seg_tile && tiles && top_k > 0 && R / top_k < (1 << kTokenBits) &&
                     tile_tokens > kPackedTokens;
    if (!tiles || top_k < 1) tile_tok = nullptr;
    if (!pack && !tile_tok) seg_tile = nullptr;
    const size_t lds = sizeof(int32_t) * (n_slots + 1);
    hipLaunchKernelGGL(dispatch_count_kernel, dim3(1), dim3(kDispatchThreads), lds, st, route_slot, R,
                       n_slots, n_shared_tokens, tile_tokens, seg_start, tiles, n_tiles, max_tiles, route_pos,
                       seg_tile, pack);
    *place = PlaceArgs{route_slot, R, n_slots, seg_start, sorted_route, route_pos, seg_tile, tiles, max_tiles,
                       top_k > 0 ? top_k : 1, pack, tile_tok, tile_tokens};
    return hipGetLastError();
}

hipError_t launch_dispatch(const int32_t *route_slot, int R, int n_slots, int n_shared_tokens,
                           int tile_tokens, int32_t *seg_start, int32_t *sorted_route,
                           int32_t *route_pos, int32_t *tiles, int32_t *n_tiles, int max_tiles,
                           hipStream_t st, int32_t *seg_tile, int top_k, bool pack_small, int32_t *tile_tok) {
    PlaceArgs a;
    hipError_t e = launch_dispatch_count(route_slot, R, n_slots, n_shared_tokens, tile_tokens, seg_start,
                                         sorted_route, route_pos, tiles, n_tiles, max_tiles, st, seg_tile, top_k,
                                         pack_small, tile_tok, &a);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(dispatch_place_kernel, dim3((n_slots + kPlaceSlotsPerBlock - 1) / kPlaceSlotsPerBlock),
                       dim3(64 * kPlaceSlotsPerBlock), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_route_slots(const int32_t *idx, int R, int E, const int32_t *slot_of_expert,
                              int n_slots, int32_t *route_slot, hipStream_t st) {
    hipLaunchKernelGGL(route_slots_kernel, dim3((R + 255) / 256), dim3(256), 0, st, idx, R, E,
                       slot_of_expert, n_slots, route_slot);
    return hipGetLastError();
}

hipError_t launch_combine(const uint16_t *y, const int32_t *route_pos, const uint16_t *shared_y,
                          const float *weights, int tokens, int top_k, int d, int mode, bool bf16,
                          uint16_t *out, hipStream_t st) {
    const bool vec = d % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(shared_y) |
                       reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (vec) {
        dim3 grid((d / 8 + 255) / 256, tokens);
        if (bf16)
            hipLaunchKernelGGL(combine8_kernel<true>, grid, dim3(256), 0, st, y, route_pos, shared_y, weights,
                               tokens, top_k, d, mode, out);
        else
            hipLaunchKernelGGL(combine8_kernel<false>, grid, dim3(256), 0, st, y, route_pos, shared_y, weights,
                               tokens, top_k, d, mode, out);
        return hipGetLastError();
    }
    dim3 grid((d + 255) / 256, tokens);
    if (bf16)
        hipLaunchKernelGGL(combine_kernel<true>, grid, dim3(256), 0, st, y, route_pos, shared_y, weights,
                           tokens, top_k, d, mode, out);
    else
        hipLaunchKernelGGL(combine_kernel<false>, grid, dim3(256), 0, st, y, route_pos, shared_y, weights,
                           tokens, top_k, d, mode, out);
    return hipGetLastError();
}

hipError_t launch_combine_routes(const void *y, int y_type, const int32_t *route_pos,
                                 const uint16_t *shared_y, const float *weights, int tokens, int top_k,
                                 int d, int mode, bool bf16, uint16_t *out, hipStream_t st) {
    dim3 grid((d + 255) / 256, tokens);
#define LOCALI_COMBINE_ROUTES(YT, B)                                                                   \
    hipLaunchKernelGGL((combine_routes_kernel<YT, B>), grid, dim3(256), 0, st, y, route_pos, shared_y, \
                       weights, top_k, d, mode, out)
    if (bf16) {
        if (y_type == 0) LOCALI_COMBINE_ROUTES(0, true);
        else if (y_type == 1) LOCALI_COMBINE_ROUTES(1, true);
        else LOCALI_COMBINE_ROUTES(2, true);
    } else {
        if (y_type == 0) LOCALI_COMBINE_ROUTES(0, false);
        else if (y_type == 1) LOCALI_COMBINE_ROUTES(1, false);
        else LOCALI_COMBINE_ROUTES(2, false);
    }
#undef LOCALI_COMBINE_ROUTES
    return hipGetLastError();
}

}  // namespace locali
