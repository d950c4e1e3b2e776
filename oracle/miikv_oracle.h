/*
 * miikv CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference runtime's CPU path for the quantized
 * KV-cache hot path.  It is the checker the GPU kernels are compared against:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  The product library (libmiikv) never links or calls it.
 *
 * Every function cites the reference file:line it follows (paths are relative
 * to the reference checkout).  All caches here are CANONICAL (row-major):
 *   codes  [kv_heads][length][head_dim]        int8
 *   scales [kv_heads][length][head_dim / 32]   fp16 bits
 * which is the reference's [head][pos][dim] layout (src/qwen3_layer.cpp:218-231,
 * include/miinfer/prefill_v2/kv_cache.hpp:24-46) with the per-row scale replaced
 * by one scale per 32-value block.
 *
 * Pinning status of each function is listed in oracle/README.md.
 */
#ifndef MIIKV_ORACLE_H
#define MIIKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIIKV_ORACLE_QBLOCK 32

/* fp32 -> fp16 bits, round-to-nearest-even with subnormals, overflow to inf,
 * NaN kept quiet.  Follows src/qwen3_layer.cpp:27-60 (float_to_half_bits_rn). */
uint16_t miikv_oracle_f32_to_f16(float value);

/* fp16 bits -> fp32, exact.  Follows src/qwen3_primitives.cpp:67-91. */
float miikv_oracle_f16_to_f32(uint16_t bits);

/* Quantize one block of 32 values with the reference device rule
 * (gfx906/kernels/qwen3_primitives.hip:7285-7322) applied per 32-value block:
 *   amax = max|x|; scale = amax > 0 ? amax/127 : 1; inv = scale > 0 ? 1/scale : 1;
 *   q = clamp(rint(x * inv), -128, 127); scale_h = fp16_rn(scale). */
void miikv_oracle_q8_0_block(const float* x, int8_t* codes, uint16_t* scale_bits);

/* Quantize n_rows rows of head_dim fp32 values per 32-value block (same rule). */
void miikv_oracle_quantize_rows_f32(const float* rows, size_t n_rows, uint32_t head_dim, int8_t* codes,
                                    uint16_t* scales);

/* K prologue of the reference store kernel for one row of head_dim values
 * (gfx906/kernels/qwen3_primitives.hip:7257-7281 with the RoPE pair of :622-659):
 *   y = x * (1 / sqrt(sum(x^2)/head_dim + eps)) * w;
 *   for i < 32: a = position * s^i with s = powf(theta, -2/64) accumulated by
 *   repeated fp32 multiplication; (y_i, y_{i+32}) <- (y_i cos a - y_{i+32} sin a,
 *   y_i sin a + y_{i+32} cos a).  Dims >= 64 are only normalised. */
void miikv_oracle_rope_sincos(float a, float* s, float* c);
void miikv_oracle_k_norm_rope(const float* x, const float* w, uint32_t head_dim, uint32_t position, float theta,
                              float eps, float* out);

/* One Q8_1 block (36 bytes: fp16 d, fp16 s, int8 qs[32]) from 32 values, as the
 * reference decode combine emits it (qwen3_primitives.hip:2354-2384):
 *   d = amax/127; inv = d != 0 ? 1/d : 0; q = clamp(roundf(x*inv), -127, 127)
 *   (round half away from zero); s = fp16(sum(q) * d). */
void miikv_oracle_q8_1_block(const float* x, uint8_t* block36);

/* Quantize n_rows rows of head_dim fp16 values (head_dim % 32 == 0). */
void miikv_oracle_quantize_rows_f16(const uint16_t* rows, size_t n_rows, uint32_t head_dim,
                                    int8_t* codes, uint16_t* scales);

/* Dequantize canonical rows: x = float(code) * float(scale_h).
 * Follows src/prefill_v2/kv_cache.cpp:161-169. */
void miikv_oracle_dequantize_rows(const int8_t* codes, const uint16_t* scales, size_t n_rows,
                                  uint32_t head_dim, float* out);

/* Softmax with a double-precision denominator.
 * Follows src/qwen3_primitives.cpp:137-146 (softmax_reference). In-place allowed. */
void miikv_oracle_softmax(const float* in, float* out, size_t n);

/* Single-query GQA attention over fp32 K/V for one query position.
 * Follows src/qwen3_layer.cpp:350-388: fp32 sequential dot, score = dot * scale
 * (the reference host divides by sqrt(head_dim); the kernels multiply by a
 * caller scale, qwen3_primitives.hip:7437-7443), softmax with a double
 * denominator (src/qwen3_primitives.cpp:137-146), fp32 weighted sum,
 * GQA map kv = h / (q_heads / kv_heads).
 *   q      [q_heads][head_dim]
 *   k, v   [kv_heads][stride_len][head_dim] (positions 0..length-1 used)
 *   out    [q_heads][head_dim]
 * gate (nullable, [q_heads][head_dim]) multiplies the output by sigmoid(gate)
 * (qwen3_primitives.hip:2362-2366). */
void miikv_oracle_attention_f32(const float* q, const float* k, const float* v,
                                uint32_t length, uint32_t stride_len,
                                uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                                float scale, const float* gate, float* out);

/* Same over a canonical q8_0 cache (dequantized with the rule above). */
void miikv_oracle_attention_q8(const float* q,
                               const int8_t* k_codes, const uint16_t* k_scales,
                               const int8_t* v_codes, const uint16_t* v_scales,
                               uint32_t length, uint32_t stride_len,
                               uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                               float scale, const float* gate, float* out);

/* Causal suffix attention: token t of a token_count-long suffix sits at absolute
 * position base_position + t and attends to cache positions [0, base_position + t].
 * The cache already holds the appended suffix rows (qwen3_primitives.hip:6826-6836).
 *   q   [token_count][q_heads][head_dim]
 *   out [token_count][q_heads][head_dim] */
void miikv_oracle_suffix_attention_q8(const float* q,
                                      const int8_t* k_codes, const uint16_t* k_scales,
                                      const int8_t* v_codes, const uint16_t* v_scales,
                                      uint32_t base_position, uint32_t token_count,
                                      uint32_t stride_len,
                                      uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                                      float scale, const float* gate, float* out);

/* 64-bit FNV-1a over u32 tokens, each widened to u64 before the xor.
 * Follows include/miinfer/prefill_v2/reusable_context.hpp:38-45. */
uint64_t miikv_oracle_token_hash(const uint32_t* tokens, size_t count);

/* Timing helper for the CPU baseline: runs miikv_oracle_attention_q8 `reps`
 * times with query heads split across `threads` pthreads; returns the median
 * seconds per call. */
double miikv_oracle_time_attention_q8(const float* q,
                                      const int8_t* k_codes, const uint16_t* k_scales,
                                      const int8_t* v_codes, const uint16_t* v_scales,
                                      uint32_t length, uint32_t stride_len,
                                      uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                                      float scale, float* out, int threads, int warmup, int reps);

#ifdef __cplusplus
}
#endif

#endif
