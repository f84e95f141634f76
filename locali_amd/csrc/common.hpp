// Shared device helpers for the streamed-MoE kernels (gfx950 / CDNA4, wave64).
//
// 16-bit activations and affine metadata travel as raw uint16 bit patterns;
// the template flag BF16 selects bfloat16 (true) or IEEE half (false).
//
// Affine weights use the MLX layout (value j of a row in word j*bits/32, LSB
// first; reference dsv4_kernels.py:26-29, 59-73). A lane streams 16-byte
// chunks of a row. Each 32-bit word is turned into packed 16-bit pairs by one
// v_and_or_b32 against a "magic" exponent (bf16 128.0 = 0x4300 or fp16
// 1024.0 = 0x6400) whose mantissa ulp is 1: a 2- or 4-bit field OR-ed into the
// low mantissa bits reads as magic + field. A field sitting 2j bits up reads
// as magic + 4^j q, so several fields are taken per shift and the matching
// activations are pre-scaled by 4^-j (exact in 16-bit floats). One v_dot2
// then accumulates x'.(magic + 4^j q) into fp32, and the per-group constant
// magic * sum(x') is subtracted once per group:
//     sum_k x_k q_k = D - magic * sum_k x'_k
// which is the factorised affine dot of dsv4_kernels.py:75-79
//     scale * sum(x q) + bias * sum(x).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace locali {

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_float(uint16_t u) {
    return __uint_as_float(static_cast<uint32_t>(u) << 16);
}

__device__ __forceinline__ uint16_t float_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_float(uint16_t u) {
    return static_cast<float>(__builtin_bit_cast(_Float16, u));
}

__device__ __forceinline__ uint16_t float_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <bool BF16>
__device__ __forceinline__ float to_float(uint16_t u) {
    if constexpr (BF16) return bf16_to_float(u);
    else return f16_to_float(u);
}

template <bool BF16>
__device__ __forceinline__ uint16_t from_float(float f) {
    if constexpr (BF16) return float_to_bf16(f);
    else return float_to_f16(f);
}

template <bool BF16>
__device__ __forceinline__ float round16(float f) {
    return to_float<BF16>(from_float<BF16>(f));
}

// fp32 += dot(a.lo*b.lo + a.hi*b.hi) over packed 16-bit pairs.
template <bool BF16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (BF16)
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                               __builtin_bit_cast(bf16x2_t, b), c, false);
    else
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a),
                                      __builtin_bit_cast(f16x2_t, b), c, false);
}

// ---------------------------------------------------------------------------
// Per-word pair tables.
//
// For each pair p of a 32-bit word: shift applied to the word, the mask that
// selects one field in each 16-bit half, the values (index within the word)
// the two fields belong to, and log2 of the factor that turns the field into
// the value's contribution (x' = x * 2^xexp). For 8-bit codes under bf16 the
// byte is split into nibbles (hi nibble weight 16, xexp = +4).
// ---------------------------------------------------------------------------
struct PairSpec {
    uint8_t shift;
    uint32_t mask;
    uint8_t lo_val, hi_val;
    int8_t lo_xexp, hi_xexp;
};

template <int BITS, bool BF16> struct Pairs;

// 2-bit, bf16 magic 128: fields 0,2,4 of the mantissa; shifts 0, 6, 12.
template <> struct Pairs<2, true> {
    static constexpr bool kSubtract = false;  // magic removed per group
    static constexpr int kCount = 8;
    static constexpr uint32_t kMagic = 0x43004300u;
    static constexpr float kMagicValue = 128.0f;
    static constexpr PairSpec kSpec[8] = {
        {0, 0x00030003u, 0, 8, 0, 0},   {0, 0x000C000Cu, 1, 9, -2, -2},
        {0, 0x00300030u, 2, 10, -4, -4}, {6, 0x00030003u, 3, 11, 0, 0},
        {6, 0x000C000Cu, 4, 12, -2, -2}, {6, 0x00300030u, 5, 13, -4, -4},
        {12, 0x00030003u, 6, 14, 0, 0}, {12, 0x000C000Cu, 7, 15, -2, -2}};
};

// 2-bit, fp16 magic 1024: fields 0,2,4,6,8; shifts 0, 10.
template <> struct Pairs<2, false> {
    static constexpr bool kSubtract = true;   // magic removed by v_pk_add_f16
    static constexpr int kCount = 8;
    static constexpr uint32_t kMagic = 0x64006400u;
    static constexpr float kMagicValue = 1024.0f;
    static constexpr PairSpec kSpec[8] = {
        {0, 0x00030003u, 0, 8, 0, 0},    {0, 0x000C000Cu, 1, 9, -2, -2},
        {0, 0x00300030u, 2, 10, -4, -4}, {0, 0x00C000C0u, 3, 11, -6, -6},
        {0, 0x03000300u, 4, 12, -8, -8}, {10, 0x00030003u, 5, 13, 0, 0},
        {10, 0x000C000Cu, 6, 14, -2, -2}, {10, 0x00300030u, 7, 15, -4, -4}};
};

// 4-bit, bf16 magic 128: only bits 0-3 fit; shifts 0, 4, 8, 12.
template <> struct Pairs<4, true> {
    static constexpr bool kSubtract = false;  // magic removed per group
    static constexpr int kCount = 4;
    static constexpr uint32_t kMagic = 0x43004300u;
    static constexpr float kMagicValue = 128.0f;
    static constexpr PairSpec kSpec[4] = {{0, 0x000F000Fu, 0, 4, 0, 0},
                                          {4, 0x000F000Fu, 1, 5, 0, 0},
                                          {8, 0x000F000Fu, 2, 6, 0, 0},
                                          {12, 0x000F000Fu, 3, 7, 0, 0}};
};

// 4-bit, fp16 magic 1024: bits 0-3 and 4-7; shifts 0, 8.
template <> struct Pairs<4, false> {
    static constexpr bool kSubtract = true;   // magic removed by v_pk_add_f16
    static constexpr int kCount = 4;
    static constexpr uint32_t kMagic = 0x64006400u;
    static constexpr float kMagicValue = 1024.0f;
    static constexpr PairSpec kSpec[4] = {{0, 0x000F000Fu, 0, 4, 0, 0},
                                          {0, 0x00F000F0u, 1, 5, -4, -4},
                                          {8, 0x000F000Fu, 2, 6, 0, 0},
                                          {8, 0x00F000F0u, 3, 7, -4, -4}};
};

// 3-bit codes split over a word's halves (spread3_halves: values 0-3 in bits
// 0-11 and 4-7 in bits 16-27, three bits each; bits 12-15 of each half are
// not read): shifts 0, 3, 6, 9, the 4-bit order and unscaled activations.
template <> struct Pairs<3, true> {
    static constexpr bool kSubtract = false;  // magic removed per group
    static constexpr int kCount = 4;
    static constexpr uint32_t kMagic = 0x43004300u;
    static constexpr float kMagicValue = 128.0f;
    static constexpr PairSpec kSpec[4] = {{0, 0x00070007u, 0, 4, 0, 0},
                                          {3, 0x00070007u, 1, 5, 0, 0},
                                          {6, 0x00070007u, 2, 6, 0, 0},
                                          {9, 0x00070007u, 3, 7, 0, 0}};
};

template <> struct Pairs<3, false> {
    static constexpr bool kSubtract = true;   // magic removed by v_pk_add_f16
    static constexpr int kCount = 4;
    static constexpr uint32_t kMagic = 0x64006400u;
    static constexpr float kMagicValue = 1024.0f;
    static constexpr PairSpec kSpec[4] = {{0, 0x00070007u, 0, 4, 0, 0},
                                          {3, 0x00070007u, 1, 5, 0, 0},
                                          {6, 0x00070007u, 2, 6, 0, 0},
                                          {9, 0x00070007u, 3, 7, 0, 0}};
};

// 8-bit, bf16: a byte does not fit the 7-bit mantissa, so each byte is two
// nibble fields (the high nibble weighs 16). Values 0..3 of the word.
template <> struct Pairs<8, true> {
    static constexpr bool kSubtract = false;  // magic removed per group
    static constexpr int kCount = 4;
    static constexpr uint32_t kMagic = 0x43004300u;
    static constexpr float kMagicValue = 128.0f;
    static constexpr PairSpec kSpec[4] = {{0, 0x000F000Fu, 0, 2, 0, 0},
                                          {4, 0x000F000Fu, 0, 2, 4, 4},
                                          {8, 0x000F000Fu, 1, 3, 0, 0},
                                          {12, 0x000F000Fu, 1, 3, 4, 4}};
};

// 8-bit, fp16 magic 1024: a whole byte fits; shifts 0, 8.
template <> struct Pairs<8, false> {
    static constexpr bool kSubtract = true;   // magic removed by v_pk_add_f16
    static constexpr int kCount = 2;
    static constexpr uint32_t kMagic = 0x64006400u;
    static constexpr float kMagicValue = 1024.0f;
    static constexpr PairSpec kSpec[2] = {{0, 0x00FF00FFu, 0, 2, 0, 0},
                                          {8, 0x00FF00FFu, 1, 3, 0, 0}};
};

// (v & mask) | magic in one gfx950 v_bitop3_b32 (truth table 0xEA for
// (src0 & src1) | src2). GFX9 VOP3 encodings take no literal constants and
// read at most one SGPR, so the mask rides in an SGPR and the magic in a VGPR
// materialised once per kernel (opaque_vgpr). A builtin rather than inline
// assembly lets the compiler track the result's hazards (no padding s_nop).
__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t magic_v) {
    return __builtin_amdgcn_bitop3_b32(v, mask, magic_v, 0xEA);
}

// A VGPR holding `value` that the compiler cannot see through (so it is kept
// in one register instead of being re-materialised at every use).
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t value) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "s"(value));
    return r;
}

// Stop the instruction scheduler from moving anything across this point
// (used to keep every load of a wave issued before its arithmetic).
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Expand pair p of a packed word into two 16-bit floats. For fp16 the magic
// is removed right away with one exact packed subtraction (the result is a
// small integer times a power of two), which keeps the 1024 offset out of the
// fp32 accumulator; for bf16 the offset (128) is removed once per group.
template <int BITS, bool BF16, int p>
__device__ __forceinline__ uint32_t expand_pair(uint32_t w, uint32_t magic_v) {
    using P = Pairs<BITS, BF16>;
    constexpr PairSpec ps = P::kSpec[p];
    const uint32_t a = and_or(w >> ps.shift, ps.mask, magic_v);
    if constexpr (P::kSubtract) {
        const f16x2_t magic = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
        return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, a) + magic);
    } else {
        return a;
    }
}

// Dot of one packed word against its pre-scaled activation pairs.
template <int BITS, bool BF16>
__device__ __forceinline__ float word_dot(uint32_t w, const uint32_t *xp, float acc,
                                          uint32_t magic_v) {
    using P = Pairs<BITS, BF16>;
    static_for<0, P::kCount>([&](auto p) {
        acc = dot2<BF16>(expand_pair<BITS, BF16, decltype(p)::value>(w, magic_v), xp[p], acc);
    });
    return acc;
}

// ---------------------------------------------------------------------------
// Wave reductions.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor(float v, int m) {
    return __shfl_xor(v, m, 64);
}

// Transposed butterfly: NV partial sums per lane, summed over the LPR lanes of
// a lane group (LPR a power of two, NV <= LPR, both powers of two). Afterwards
// every lane of the group holds the total of value index
//     (lane % LPR) / (LPR / NV)
// in v[0]. Costs NV-1 + log2(LPR/NV) shuffles instead of NV*log2(LPR).
template <int NV, int LPR>
__device__ __forceinline__ void reduce_transposed(float (&v)[NV], int lane) {
    int nv = NV;
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) {
        if (nv > 1) {
            const int half = nv >> 1;
            const bool upper = (lane & m) != 0;
#pragma unroll
            for (int i = 0; i < NV / 2; ++i) {
                if (i < half) {
                    const float a = v[i], b = v[i + half];
                    const float send = upper ? a : b;
                    const float keep = upper ? b : a;
                    v[i] = keep + shfl_xor(send, m);
                }
            }
            nv = half;
        } else {
            v[0] += shfl_xor(v[0], m);
        }
    }
}

// ---- wave-wide arg-max over 64-bit keys -------------------------------------
// Monotone map of a float onto uint32 (larger float -> larger key; -inf maps
// above 0, so 0 can mark "no candidate").
__device__ __forceinline__ uint32_t ordered_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    return u ^ ((static_cast<uint32_t>(static_cast<int32_t>(u) >> 31)) | 0x80000000u);
}

template <int CTRL>
__device__ __forceinline__ uint32_t max_dpp(uint32_t v) {
    return max(v, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, false)));
}

// Maximum of v over the wave, in every lane, without leaving the vector
// unit: quad swaps (xor 1, xor 2), half-row and row mirrors (DPP) give each
// 16-lane row its maximum, then the row pairs (permlane16 swap) and the wave
// halves (permlane32 swap) meet.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max_dpp<0xB1>(v);    // quad_perm [1,0,3,2]
    v = max_dpp<0x4E>(v);    // quad_perm [2,3,0,1]
    v = max_dpp<0x141>(v);   // row_half_mirror
    v = max_dpp<0x140>(v);   // row_mirror
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max(p[0], p[1]);
    const auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max(q[0], q[1]);
}

// Maximum of the 64-bit key (hi, lo) over the wave, in every lane: the
// largest hi, then the largest lo among the lanes that hold it.
__device__ __forceinline__ void wave_max_key(uint32_t &hi, uint32_t &lo) {
    const uint32_t mh = wave_max_u32(hi);
    lo = wave_max_u32(hi == mh ? lo : 0u);
    hi = mh;
}

__device__ __forceinline__ float sigmoidf_(float g) { return 1.0f / (1.0f + __expf(-g)); }

// Clamped SwiGLU on projection outputs already rounded to the activation
// dtype (reference dsv4_arena.py:225-234): up clipped to +-L, gate capped at
// L (L <= 0 disables both), then silu(gate) * up either op by op in the
// 16-bit dtype (sigmoid, gate*sigmoid and *up each rounded) or in fp32 with
// one final rounding.
template <bool BF16>
__device__ __forceinline__ uint16_t swiglu16(float gate, float up, float limit, bool fp32_swiglu) {
    if (limit > 0.0f) {
        up = fminf(fmaxf(up, -limit), limit);
        gate = fminf(gate, limit);
    }
    if (fp32_swiglu) return from_float<BF16>(gate * sigmoidf_(gate) * up);
    const float sig = round16<BF16>(sigmoidf_(gate));
    const float act = round16<BF16>(gate * sig);
    return from_float<BF16>(act * up);
}

}  // namespace locali
