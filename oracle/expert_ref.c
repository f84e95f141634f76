/*
 * C restatement of the streamed-MoE expert arithmetic -- TEST INFRASTRUCTURE
 * ONLY. Used by tests/ as an independent checker at full sizes (where the
 * numpy fp64 oracle is slow) and by bench.py as the CPU baseline (the
 * reference's MLX-CPU path cannot run here). Never linked by the product.
 *
 * Arithmetic contract (reference dsv4_arena.py:168-235, arena.py:543-547,
 * 619-624; per-group factorised affine dot of dsv4_kernels.py:75-79):
 *   proj(v)[n] = round_T( sum_g  s[n,g] * sum_{k in g} v_k q[n,k]
 *                               + b[n,g] * sum_{k in g} v_k )      (fp32 acc)
 *   up = proj_up(x), gate = proj_gate(x); up = clip(up,+-L), gate = min(gate,L)
 *   h = round_T(round_T(gate * round_T(sigmoid(gate))) * up)
 *       or round_T(silu_f32(gate) * up) with fp32_swiglu
 *   y = proj_down(h)
 *   out[t] = round_T( sum_j round_T(y_tj * round_T(w_tj)) ) (+ shared, rounded)
 * T is bf16 (dt = 2) or fp16 (dt = 1); values travel as uint16 bit patterns.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

static float bf16_to_f(uint16_t u) {
    uint32_t v = (uint32_t)u << 16;
    float f;
    memcpy(&f, &v, 4);
    return f;
}

static uint16_t f_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float f16_to_f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff, out;
    if (exp == 0) {
        if (man == 0) out = sign;
        else {
            int e = -1;
            do { e++; man <<= 1; } while (!(man & 0x400));
            out = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ff) << 13);
        }
    } else if (exp == 31) out = sign | 0x7f800000u | (man << 13);
    else out = sign | ((exp + 127 - 15) << 23) | (man << 13);
    float f;
    memcpy(&f, &out, 4);
    return f;
}

static uint16_t f_to_f16(float f) {
    /* IEEE binary32 -> binary16, round to nearest even, with subnormals. */
    uint32_t u;
    memcpy(&u, &f, 4);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t au = u & 0x7fffffffu;
    if (au > 0x7f800000u) return sign | 0x7e00u;            /* NaN */
    if (au >= 0x477ff000u) return sign | 0x7c00u;           /* >= 65520: inf */
    if (au < 0x38800000u) {                                 /* below 2^-14 */
        if (au < 0x33000000u) return sign;                  /* < 2^-25: 0 */
        const int e = (int)(au >> 23);                      /* biased */
        uint32_t man = (au & 0x7fffffu) | 0x800000u;
        const int shift = 126 - e;                          /* 14 .. 24 */
        uint32_t half = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1u);
        const uint32_t mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1u))) half++;
        return sign | (uint16_t)half;
    }
    uint32_t v = au - 0x38000000u;                          /* rebias 127->15 */
    uint32_t half = v >> 13;
    const uint32_t rem = v & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
    return sign | (uint16_t)half;
}

static float to_f(uint16_t u, int dt) { return dt == DT_BF16 ? bf16_to_f(u) : f16_to_f(u); }
static uint16_t from_f(float f, int dt) { return dt == DT_BF16 ? f_to_bf16(f) : f_to_f16(f); }
static float round_dt(float f, int dt) { return to_f(from_f(f, dt), dt); }

typedef struct {
    const uint32_t *w;      /* slot 0 of [S, N, K*bits/32] */
    const uint16_t *s;      /* slot 0 of [S, N, K/group] */
    const uint16_t *b;
    int32_t bits, group, N, K, meta_dt;
} oracle_proj;

/* out[n] (fp32, not rounded) for one vector v of length K, slot `slot`. */
static void qmv_rows(const oracle_proj *p, int slot, const float *v, float *out,
                     int n0, int n1) {
    const int words = p->K * p->bits / 32, groups = p->K / p->group;
    const uint32_t mask = (1u << p->bits) - 1u;
    const uint32_t *W = p->w + (size_t)slot * p->N * words;
    const uint16_t *S = p->s + (size_t)slot * p->N * groups;
    const uint16_t *B = p->b + (size_t)slot * p->N * groups;
    for (int n = n0; n < n1; n++) {
        float acc = 0.f;
        for (int g = 0; g < groups; g++) {
            float dot = 0.f, vs = 0.f;
            for (int k = g * p->group; k < (g + 1) * p->group; k++) {
                /* value k starts at bit k * bits of the row's little-endian
                   stream; a 3-bit value may continue into the next word */
                const uint32_t *row = W + (size_t)n * words;
                const int off = k * p->bits, wi = off >> 5, sh = off & 31;
                uint32_t code = row[wi] >> sh;
                if (sh + p->bits > 32) code |= row[wi + 1] << (32 - sh);
                float q = (float)(code & mask);
                dot += v[k] * q;
                vs += v[k];
            }
            acc += to_f(S[(size_t)n * groups + g], p->meta_dt) * dot
                 + to_f(B[(size_t)n * groups + g], p->meta_dt) * vs;
        }
        out[n] = acc;
    }
}

void oracle_qmv(const oracle_proj *p, int slot, const float *v, float *out) {
#pragma omp parallel for schedule(static)
    for (int c = 0; c < (p->N + 63) / 64; c++) {
        int n0 = c * 64, n1 = n0 + 64 < p->N ? n0 + 64 : p->N;
        qmv_rows(p, slot, v, out, n0, n1);
    }
}

static float sigmoid_f(float g) { return 1.f / (1.f + expf(-g)); }

/* One expert on one vector. x values must already be representable in dt.
 * scratch: 3 * dff floats. y: d_model floats (rounded to dt). */
void oracle_expert(const oracle_proj *gate, const oracle_proj *up,
                   const oracle_proj *down, int slot, const float *x, int dt,
                   float limit, int fp32_swiglu, float *scratch, float *y) {
    const int dff = gate->N;
    float *g = scratch, *u = scratch + dff, *h = scratch + 2 * dff;
    oracle_qmv(up, slot, x, u);
    oracle_qmv(gate, slot, x, g);
    for (int n = 0; n < dff; n++) {
        float uu = round_dt(u[n], dt), gg = round_dt(g[n], dt);
        if (limit > 0.f) {
            uu = uu < -limit ? -limit : (uu > limit ? limit : uu);
            gg = gg > limit ? limit : gg;
        }
        if (fp32_swiglu) {
            h[n] = round_dt(gg * sigmoid_f(gg) * uu, dt);
        } else {
            float sg = round_dt(sigmoid_f(gg), dt);
            float a = round_dt(gg * sg, dt);
            h[n] = round_dt(a * uu, dt);
        }
    }
    oracle_qmv(down, slot, h, y);
    for (int n = 0; n < down->N; n++) y[n] = round_dt(y[n], dt);
}

/* Full layer on T tokens. slots [T*k] (arena slot per route), weights [T*k]
 * fp32 router weights (cast to dt here), x [T*d] values in dt. shared_* may
 * be NULL. out [T*d] values rounded to dt; terms (optional, zero-filled by
 * the caller) receives the sum of |rounded terms| added per element. */
int oracle_moe_layer(const oracle_proj *gate, const oracle_proj *up,
                     const oracle_proj *down, const oracle_proj *sgate,
                     const oracle_proj *sup, const oracle_proj *sdown,
                     const float *x, int T, int k, const int32_t *slots,
                     const float *weights, int dt, float limit,
                     int fp32_swiglu, float *out, float *terms) {
    const int d = down->N, dff = gate->N;
    float *scratch = (float *)malloc(sizeof(float) * (3 * dff + 2 * d));
    if (!scratch) return -1;
    float *y = scratch + 3 * dff, *acc = y + d;
    for (int t = 0; t < T; t++) {
        const float *xt = x + (size_t)t * d;
        for (int n = 0; n < d; n++) acc[n] = 0.f;
        for (int j = 0; j < k; j++) {
            oracle_expert(gate, up, down, slots[t * k + j], xt, dt, limit,
                          fp32_swiglu, scratch, y);
            float w = round_dt(weights[t * k + j], dt);
            for (int n = 0; n < d; n++) {
                const float term = round_dt(y[n] * w, dt);
                acc[n] += term;
                if (terms) terms[(size_t)t * d + n] += fabsf(term);
            }
        }
        for (int n = 0; n < d; n++) out[(size_t)t * d + n] = round_dt(acc[n], dt);
        if (sgate) {
            oracle_expert(sgate, sup, sdown, 0, xt, dt, limit, fp32_swiglu, scratch, y);
            for (int n = 0; n < d; n++) {
                out[(size_t)t * d + n] = round_dt(out[(size_t)t * d + n] + y[n], dt);
                if (terms) terms[(size_t)t * d + n] += fabsf(y[n]);
            }
        }
    }
    free(scratch);
    return 0;
}

/* fp32 router: logits = x . Wg (Wg given as fp32 values), score function
 * 0 = sqrtsoftplus, 1 = sigmoid; selection on score + bias (bias may be NULL),
 * top-k by descending selection, ties to the lower expert id; weights
 * renormalised (norm != 0) and scaled. */
void oracle_router(const float *x, const float *wg, const float *bias, int T,
                   int d, int E, int k, int score_func, int norm, float scale,
                   int32_t *idx, float *weights) {
    float *sc = (float *)malloc(sizeof(float) * E * 2);
    float *sel = sc + E;
    for (int t = 0; t < T; t++) {
#pragma omp parallel for schedule(static)
        for (int e = 0; e < E; e++) {
            float l = 0.f;
            for (int i = 0; i < d; i++) l += x[(size_t)t * d + i] * wg[(size_t)e * d + i];
            float s;
            if (score_func == 0) {
                float sp = l > 20.f ? l : log1pf(expf(l));
                s = sqrtf(sp);
            } else {
                s = 1.f / (1.f + expf(-l));
            }
            sc[e] = s;
            sel[e] = s + (bias ? bias[e] : 0.f);
        }
        float sum = 0.f;
        for (int j = 0; j < k; j++) {
            int best = -1;
            for (int e = 0; e < E; e++) {
                int taken = 0;
                for (int q = 0; q < j; q++) taken |= idx[t * k + q] == e;
                if (taken) continue;
                if (best < 0 || sel[e] > sel[best]) best = e;
            }
            idx[t * k + j] = best;
            weights[t * k + j] = sc[best];
            sum += sc[best];
        }
        for (int j = 0; j < k; j++) {
            float w = weights[t * k + j];
            if (norm) w = w / (sum + 1e-20f);
            weights[t * k + j] = w * scale;
        }
    }
    free(sc);
}

/* Round an fp32 array to dt and back (tests of the rounding helpers). */
void oracle_round_array(const float *in, float *out, int n, int dt) {
    for (int i = 0; i < n; i++) out[i] = round_dt(in[i], dt);
}

/* Threads of the parallel loops above (n <= 0: every processor), so the CPU
 * baseline can be timed on one core and on all of them in one process. */
void oracle_set_threads(int n) { omp_set_num_threads(n > 0 ? n : omp_get_num_procs()); }
