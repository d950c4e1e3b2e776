/*
 * miikv CPU oracle — TEST INFRASTRUCTURE ONLY (see miikv_oracle.h).
 * Compiled with -O2 -ffp-contract=off -fno-fast-math so every fp32 operation is
 * rounded exactly as written (no FMA contraction, no reassociation).
 */
#define _POSIX_C_SOURCE 200809L
#include "miikv_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* src/qwen3_layer.cpp:27-60 */
uint16_t miikv_oracle_f32_to_f16(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const uint32_t exponent = (bits >> 23) & 0xffu;
    const uint32_t mantissa = bits & 0x7fffffu;
    if (exponent == 0xffu) {
        return (uint16_t)(sign | 0x7c00u | (mantissa != 0 ? 0x0200u : 0u));
    }
    const int half_exp = (int)exponent - 127 + 15;
    if (half_exp <= 0) {
        /* Subnormal half (or zero): shift the full significand right. */
        if (half_exp < -10) return (uint16_t)sign;
        const uint32_t significand = mantissa | 0x00800000u;
        const int shift = 14 - half_exp;
        uint32_t rounded = significand >> shift;
        const uint32_t rem = significand & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (rounded & 1u))) ++rounded;
        return (uint16_t)(sign | rounded);
    }
    if (half_exp >= 31) return (uint16_t)(sign | 0x7c00u);
    uint32_t mant = mantissa >> 13;
    const uint32_t rem = mantissa & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (mant & 1u))) {
        ++mant;
        if (mant == 0x400u) {
            mant = 0;
            if (half_exp + 1 >= 31) return (uint16_t)(sign | 0x7c00u);
            return (uint16_t)(sign | ((uint32_t)(half_exp + 1) << 10));
        }
    }
    return (uint16_t)(sign | ((uint32_t)half_exp << 10) | mant);
}

/* src/qwen3_primitives.cpp:67-91 */
float miikv_oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)(h & 0x8000u)) << 16;
    const uint32_t exponent = (h >> 10) & 0x1fu;
    const uint32_t fraction = h & 0x03ffu;
    uint32_t out = sign;
    if (exponent == 0) {
        if (fraction != 0) {
            /* Normalise the subnormal: find the leading one. */
            uint32_t f = fraction;
            uint32_t shifts = 0;
            while ((f & 0x0400u) == 0) {
                f <<= 1;
                ++shifts;
            }
            f &= 0x03ffu;
            out |= (127u - 15u - shifts + 1u) << 23;
            out |= f << 13;
        }
    } else if (exponent == 0x1fu) {
        out |= 0x7f800000u | (fraction << 13);
    } else {
        out |= (exponent + 112u) << 23;
        out |= fraction << 13;
    }
    float result;
    memcpy(&result, &out, sizeof(result));
    return result;
}

/* gfx906/kernels/qwen3_primitives.hip:7285-7322, applied to one 32-value block. */
void miikv_oracle_q8_0_block(const float* x, int8_t* codes, uint16_t* scale_bits) {
    float amax = 0.0f;
    for (int i = 0; i < MIIKV_ORACLE_QBLOCK; ++i) {
        const float a = fabsf(x[i]);
        amax = a > amax ? a : amax; /* fmaxf semantics for finite inputs */
    }
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 1.0f;
    for (int i = 0; i < MIIKV_ORACLE_QBLOCK; ++i) {
        const float prod = x[i] * inv;
        long r = lrintf(prod); /* round-half-even in the default rounding mode */
        if (r < -128) r = -128;
        if (r > 127) r = 127;
        codes[i] = (int8_t)r;
    }
    *scale_bits = miikv_oracle_f32_to_f16(scale);
}

void miikv_oracle_quantize_rows_f16(const uint16_t* rows, size_t n_rows, uint32_t head_dim,
                                    int8_t* codes, uint16_t* scales) {
    const uint32_t nblk = head_dim / MIIKV_ORACLE_QBLOCK;
    float block[MIIKV_ORACLE_QBLOCK];
    for (size_t r = 0; r < n_rows; ++r) {
        for (uint32_t b = 0; b < nblk; ++b) {
            const uint16_t* src = rows + r * head_dim + (size_t)b * MIIKV_ORACLE_QBLOCK;
            for (int i = 0; i < MIIKV_ORACLE_QBLOCK; ++i) block[i] = miikv_oracle_f16_to_f32(src[i]);
            miikv_oracle_q8_0_block(block, codes + r * head_dim + (size_t)b * MIIKV_ORACLE_QBLOCK,
                                    scales + r * nblk + b);
        }
    }
}

void miikv_oracle_quantize_rows_f32(const float* rows, size_t n_rows, uint32_t head_dim, int8_t* codes,
                                    uint16_t* scales) {
    const uint32_t nblk = head_dim / MIIKV_ORACLE_QBLOCK;
    for (size_t r = 0; r < n_rows; ++r)
        for (uint32_t b = 0; b < nblk; ++b)
            miikv_oracle_q8_0_block(rows + r * head_dim + (size_t)b * MIIKV_ORACLE_QBLOCK,
                                    codes + r * head_dim + (size_t)b * MIIKV_ORACLE_QBLOCK, scales + r * nblk + b);
}

/* sin and cos of a RoPE angle with the float arithmetic of the library's prologue
 * (miinfer_amd/csrc/miikv_rope.h, rope_sincos): Cody-Waite reduction by pi/2 in three
 * parts with fused multiply-adds, Taylor polynomials on [-pi/4, pi/4], quadrant.  The
 * reference calls cosf / sinf (qwen3_primitives.hip:651-652); this pair is pinned
 * against float64 sin / cos in the tests (within two ulps). */
void miikv_oracle_rope_sincos(float a, float* s, float* c) {
    const float k = rintf(a * 6.366197467e-01f);
    float r = fmaf(-k, 1.5703125f, a);
    r = fmaf(-k, 4.838267923e-04f, r);
    r = fmaf(-k, 2.563282919e-12f, r);
    const float r2 = r * r;
    float ps = fmaf(r2, -2.505210794e-08f, 2.755731884e-06f);
    ps = fmaf(r2, ps, -1.984127011e-04f);
    ps = fmaf(r2, ps, 8.333333768e-03f);
    ps = fmaf(r2, ps, -1.666666716e-01f);
    const float sr = fmaf(r * r2, ps, r);
    float pc = fmaf(r2, 2.087675588e-09f, -2.755731998e-07f);
    pc = fmaf(r2, pc, 2.480158764e-05f);
    pc = fmaf(r2, pc, -1.388888923e-03f);
    pc = fmaf(r2, pc, 4.166666791e-02f);
    pc = fmaf(r2, pc, -5.000000000e-01f);
    const float cr = fmaf(r2, pc, 1.0f);
    const int q = (int)k & 3;
    *s = q == 0 ? sr : q == 1 ? cr : q == 2 ? -sr : -cr;
    *c = q == 0 ? cr : q == 1 ? -sr : q == 2 ? -cr : sr;
}

/* gfx906/kernels/qwen3_primitives.hip:7257-7281 (RMSNorm * weight, RoPE on dims
 * 0..63) and :622-659 (compute_qwen35_rope_pair: every pair < 32 falls in a
 * rotated section, and the three section angles are the same position). */
void miikv_oracle_k_norm_rope(const float* x, const float* w, uint32_t head_dim, uint32_t position, float theta,
                              float eps, float* out) {
    /* sum of squares in the reference's LDS tree order (qwen3_primitives.hip:7257-7263):
     * p[t] = x[t]^2, then p[t] += p[t + stride] for stride = D/2, D/4, ..., 1 */
    float p[512];
    for (uint32_t d = 0; d < head_dim; ++d) p[d] = x[d] * x[d];
    for (uint32_t stride = head_dim / 2; stride > 0; stride /= 2)
        for (uint32_t t = 0; t < stride; ++t) p[t] += p[t + stride];
    const float ss = p[0];
    /* the reference takes rsqrtf (a hardware approximation within one ulp of this) */
    const float r = 1.0f / sqrtf(ss / (float)head_dim + eps);
    for (uint32_t d = 0; d < head_dim; ++d) out[d] = x[d] * r * w[d];
    const float step = powf(theta, -2.0f / 64.0f);
    float angle = (float)position;
    for (uint32_t i = 0; i < 32; ++i) {
        float s, c;
        miikv_oracle_rope_sincos(angle, &s, &c);
        const float x0 = out[i], x1 = out[i + 32];
        out[i] = x0 * c - x1 * s;
        out[i + 32] = x0 * s + x1 * c;
        angle *= step;
    }
}

/* gfx906/kernels/qwen3_primitives.hip:2354-2384; block layout
 * include/miinfer/q4_q8_gemv.hpp:23-27. */
void miikv_oracle_q8_1_block(const float* x, uint8_t* block36) {
    float amax = 0.0f;
    for (int i = 0; i < MIIKV_ORACLE_QBLOCK; ++i) {
        const float a = fabsf(x[i]);
        amax = a > amax ? a : amax;
    }
    const float d = amax / 127.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    int sum = 0;
    for (int i = 0; i < MIIKV_ORACLE_QBLOCK; ++i) {
        long q = lroundf(x[i] * inv); /* half away from zero, as roundf */
        if (q < -127) q = -127;
        if (q > 127) q = 127;
        block36[4 + i] = (uint8_t)(int8_t)q;
        sum += (int)q;
    }
    const uint16_t db = miikv_oracle_f32_to_f16(d);
    const uint16_t sb = miikv_oracle_f32_to_f16((float)sum * d);
    block36[0] = (uint8_t)(db & 0xff);
    block36[1] = (uint8_t)(db >> 8);
    block36[2] = (uint8_t)(sb & 0xff);
    block36[3] = (uint8_t)(sb >> 8);
}

/* src/prefill_v2/kv_cache.cpp:161-169 */
void miikv_oracle_dequantize_rows(const int8_t* codes, const uint16_t* scales, size_t n_rows,
                                  uint32_t head_dim, float* out) {
    const uint32_t nblk = head_dim / MIIKV_ORACLE_QBLOCK;
    for (size_t r = 0; r < n_rows; ++r) {
        for (uint32_t d = 0; d < head_dim; ++d) {
            const float s = miikv_oracle_f16_to_f32(scales[r * nblk + d / MIIKV_ORACLE_QBLOCK]);
            out[r * head_dim + d] = (float)codes[r * head_dim + d] * s;
        }
    }
}

/* src/qwen3_primitives.cpp:137-146: max-shifted exp with a double denominator. */
void miikv_oracle_softmax(const float* in, float* out, size_t n) {
    if (n == 0) return;
    float maximum = in[0];
    for (size_t p = 1; p < n; ++p) maximum = in[p] > maximum ? in[p] : maximum;
    double denom = 0.0;
    for (size_t p = 0; p < n; ++p) denom += exp((double)(in[p] - maximum));
    for (size_t p = 0; p < n; ++p) out[p] = (float)(exp((double)(in[p] - maximum)) / denom);
}

/* One query head: src/qwen3_layer.cpp:350-388 with the softmax above. */
static void attend_one_head(const float* qh, const float* kh, const float* vh, uint32_t length,
                            uint32_t head_dim, float scale, const float* gh, float* oh,
                            float* scores) {
    for (uint32_t p = 0; p < length; ++p) {
        const float* kr = kh + (size_t)p * head_dim;
        float dot = 0.0f;
        for (uint32_t i = 0; i < head_dim; ++i) dot += qh[i] * kr[i];
        scores[p] = dot * scale;
    }
    miikv_oracle_softmax(scores, scores, length);
    for (uint32_t i = 0; i < head_dim; ++i) {
        float acc = 0.0f;
        for (uint32_t p = 0; p < length; ++p) acc += scores[p] * vh[(size_t)p * head_dim + i];
        if (gh != NULL) acc = acc * (1.0f / (1.0f + expf(-gh[i])));
        oh[i] = acc;
    }
}

void miikv_oracle_attention_f32(const float* q, const float* k, const float* v,
                                uint32_t length, uint32_t stride_len,
                                uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                                float scale, const float* gate, float* out) {
    if (length == 0) {
        memset(out, 0, sizeof(float) * q_heads * head_dim);
        return;
    }
    float* scores = (float*)malloc(sizeof(float) * length);
    const uint32_t group = q_heads / kv_heads;
    for (uint32_t h = 0; h < q_heads; ++h) {
        const size_t kv = (size_t)(h / group) * stride_len * head_dim;
        attend_one_head(q + (size_t)h * head_dim, k + kv, v + kv, length, head_dim, scale,
                        gate ? gate + (size_t)h * head_dim : NULL, out + (size_t)h * head_dim,
                        scores);
    }
    free(scores);
}

/* Dequantize positions [0, length) of every kv head into a compact fp32 copy. */
static void dequant_cache(const int8_t* codes, const uint16_t* scales, uint32_t length,
                          uint32_t stride_len, uint32_t kv_heads, uint32_t head_dim, float* out) {
    const uint32_t nblk = head_dim / MIIKV_ORACLE_QBLOCK;
    for (uint32_t h = 0; h < kv_heads; ++h) {
        miikv_oracle_dequantize_rows(codes + (size_t)h * stride_len * head_dim,
                                     scales + (size_t)h * stride_len * nblk, length, head_dim,
                                     out + (size_t)h * length * head_dim);
    }
}

void miikv_oracle_attention_q8(const float* q,
                               const int8_t* k_codes, const uint16_t* k_scales,
                               const int8_t* v_codes, const uint16_t* v_scales,
                               uint32_t length, uint32_t stride_len,
                               uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                               float scale, const float* gate, float* out) {
    const size_t n = (size_t)kv_heads * length * head_dim;
    float* k = (float*)malloc(sizeof(float) * (n ? n : 1));
    float* v = (float*)malloc(sizeof(float) * (n ? n : 1));
    dequant_cache(k_codes, k_scales, length, stride_len, kv_heads, head_dim, k);
    dequant_cache(v_codes, v_scales, length, stride_len, kv_heads, head_dim, v);
    miikv_oracle_attention_f32(q, k, v, length, length, q_heads, kv_heads, head_dim, scale, gate,
                               out);
    free(k);
    free(v);
}

void miikv_oracle_suffix_attention_q8(const float* q,
                                      const int8_t* k_codes, const uint16_t* k_scales,
                                      const int8_t* v_codes, const uint16_t* v_scales,
                                      uint32_t base_position, uint32_t token_count,
                                      uint32_t stride_len,
                                      uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                                      float scale, const float* gate, float* out) {
    const uint32_t total = base_position + token_count;
    const size_t n = (size_t)kv_heads * total * head_dim;
    float* k = (float*)malloc(sizeof(float) * (n ? n : 1));
    float* v = (float*)malloc(sizeof(float) * (n ? n : 1));
    dequant_cache(k_codes, k_scales, total, stride_len, kv_heads, head_dim, k);
    dequant_cache(v_codes, v_scales, total, stride_len, kv_heads, head_dim, v);
    float* scores = (float*)malloc(sizeof(float) * (total ? total : 1));
    const uint32_t group = q_heads / kv_heads;
    for (uint32_t t = 0; t < token_count; ++t) {
        const uint32_t length = base_position + t + 1;
        for (uint32_t h = 0; h < q_heads; ++h) {
            const size_t row = ((size_t)t * q_heads + h) * head_dim;
            const size_t kv = (size_t)(h / group) * total * head_dim;
            attend_one_head(q + row, k + kv, v + kv, length, head_dim, scale,
                            gate ? gate + row : NULL, out + row, scores);
        }
    }
    free(scores);
    free(k);
    free(v);
}

/* include/miinfer/prefill_v2/reusable_context.hpp:38-45 */
uint64_t miikv_oracle_token_hash(const uint32_t* tokens, size_t count) {
    uint64_t hash = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < count; ++i) {
        hash ^= (uint64_t)tokens[i];
        hash *= 0x100000001b3ull;
    }
    return hash;
}

/* ---- CPU-baseline timing (threads split the query heads) ---------------- */

typedef struct {
    const float* q;
    const float* k;
    const float* v;
    uint32_t length, q_heads, kv_heads, head_dim, h0, h1;
    float scale;
    float* out;
} worker_arg;

static void* worker(void* p) {
    worker_arg* a = (worker_arg*)p;
    float* scores = (float*)malloc(sizeof(float) * a->length);
    const uint32_t group = a->q_heads / a->kv_heads;
    for (uint32_t h = a->h0; h < a->h1; ++h) {
        const size_t kv = (size_t)(h / group) * a->length * a->head_dim;
        attend_one_head(a->q + (size_t)h * a->head_dim, a->k + kv, a->v + kv, a->length,
                        a->head_dim, a->scale, NULL, a->out + (size_t)h * a->head_dim, scores);
    }
    free(scores);
    return NULL;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static int cmp_double(const void* a, const void* b) {
    const double x = *(const double*)a, y = *(const double*)b;
    return (x > y) - (x < y);
}

double miikv_oracle_time_attention_q8(const float* q,
                                      const int8_t* k_codes, const uint16_t* k_scales,
                                      const int8_t* v_codes, const uint16_t* v_scales,
                                      uint32_t length, uint32_t stride_len,
                                      uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                                      float scale, float* out, int threads, int warmup, int reps) {
    if (threads < 1) threads = 1;
    if ((uint32_t)threads > q_heads) threads = (int)q_heads;
    if (reps < 1) reps = 1;
    double* times = (double*)malloc(sizeof(double) * (size_t)reps);
    pthread_t* tids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    worker_arg* args = (worker_arg*)malloc(sizeof(worker_arg) * (size_t)threads);
    const size_t n = (size_t)kv_heads * length * head_dim;
    float* k = (float*)malloc(sizeof(float) * n);
    float* v = (float*)malloc(sizeof(float) * n);
    /* The reference CPU path attends over an fp32 [head][pos][dim] cache
     * (src/qwen3_layer.cpp:218-231, 350-388): dequantise once, outside timing. */
    dequant_cache(k_codes, k_scales, length, stride_len, kv_heads, head_dim, k);
    dequant_cache(v_codes, v_scales, length, stride_len, kv_heads, head_dim, v);
    for (int it = 0; it < warmup + reps; ++it) {
        const double t0 = now_s();
        for (int t = 0; t < threads; ++t) {
            worker_arg* a = &args[t];
            a->q = q; a->k = k; a->v = v; a->length = length; a->q_heads = q_heads;
            a->kv_heads = kv_heads; a->head_dim = head_dim; a->scale = scale; a->out = out;
            a->h0 = (uint32_t)((uint64_t)q_heads * (uint64_t)t / (uint64_t)threads);
            a->h1 = (uint32_t)((uint64_t)q_heads * (uint64_t)(t + 1) / (uint64_t)threads);
            if (threads == 1) worker(a);
            else pthread_create(&tids[t], NULL, worker, a);
        }
        if (threads > 1)
            for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
        const double dt = now_s() - t0;
        if (it >= warmup) times[it - warmup] = dt;
    }
    qsort(times, (size_t)reps, sizeof(double), cmp_double);
    const double med = times[reps / 2];
    free(times); free(tids); free(args); free(k); free(v);
    return med;
}
