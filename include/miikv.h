/*
 * miikv — MI355X-native (gfx950) quantized KV-cache path: C ABI.
 *
 * Launch-only, asynchronous entry points with plain pointers and sizes.  The
 * caller owns every device buffer (including the workspace); no launch entry
 * point allocates device memory.  The exceptions are the host-synchronous file
 * calls miikv_session_save / miikv_session_load, which stage one layer through
 * a device buffer they allocate and free (documented at each).  Each entry
 * point returns a miikv_status: 0 on success, > 0 for an invalid argument
 * (nothing was launched), < 0 for a HIP error (the negated hipError_t).  The reference aborts the process on invalid
 * arguments (include/miinfer/hip_check.hpp:11-38); this ABI reports instead.
 *
 * Streams are passed as `void*` holding a hipStream_t (NULL = default stream).
 * Device-state pointers (miikv_decode_state / miikv_prefill_state) live in
 * device memory and are read by the kernels, so calls that take them can be
 * captured into a HIP graph and replayed while the position advances on the
 * device, as the reference does (include/miinfer/qwen3_gpu_primitives.hpp:30-45).
 *
 * ---------------------------------------------------------------------------
 * Cache layout in HBM (q8_0: 32-value blocks, one fp16 scale per block)
 * ---------------------------------------------------------------------------
 * The cache is a set of pages of `page_tokens` tokens (a multiple of 64).  A
 * CONTIGUOUS cache is the special case of a single page whose page_tokens is the
 * capacity: its slabs are ordered [kv_head][capacity] like the reference's
 * planes (include/miinfer/prefill_v2/kv_cache.hpp:24-46), but the bytes inside a
 * slab are tiled as below, not [capacity][head_dim] row-major, so code that
 * reads or writes the raw planes must go through miikv_export_canonical /
 * miikv_import_canonical (or miikv_export_dequant).  A PAGED cache maps
 * logical page i of sequence b to physical page block_table[b*table_stride + i].
 *
 * Each of the four planes is [page][kv_head][slab]; one slab holds page_tokens
 * tokens of one kv head:
 *   k_scales, v_scales slab: [page_tokens][head_dim/32] fp16 (row-major)
 *   k_codes slab (int8), MFMA-A-operand tiling in 16-token tiles:
 *       token t = 16*T + m, dim d = 64*c + 32*e + 8*g + j  (m<16, e<2, g<4, j<8)
 *       byte offset = T*(16*head_dim) + c*1024 + g*256 + m*16 + e*8 + j
 *   v_codes slab (int8), token-contiguous per dim in 32-token groups:
 *       token t = 32*H + 16*J + 4*G + I  (J<2, G<4, I<4)
 *       byte offset = H*(32*head_dim) + d*32 + G*8 + J*4 + I
 * miikv_export_canonical() converts any token range back to row-major codes.
 */
#ifndef MIIKV_H
#define MIIKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIIKV_ABI_VERSION 1u
#define MIIKV_QBLOCK 32u

typedef int miikv_status;
enum {
    MIIKV_OK = 0,
    MIIKV_EINVAL = 1,       /* invalid argument: nothing launched */
    MIIKV_EUNSUPPORTED = 2, /* valid but not implemented (e.g. head_dim 64) */
    MIIKV_EWORKSPACE = 3,   /* workspace missing or too small */
};

enum { MIIKV_LAYOUT_CONTIGUOUS = 0, MIIKV_LAYOUT_PAGED = 1 };

/* Mirrors KvCacheQuantMode (include/miinfer/prefill_v2/kv_cache.hpp:16-21).
 * A q8 plane (K or V) holds int8 codes plus one fp16 scale per 32 values; an fp16
 * plane holds the fp16 rows themselves in the same tiled element order (2 bytes per
 * element, twice the bytes of a q8 code plane) and has no scales (its scale pointer
 * may be NULL).  Every mode is accepted by append, decode, suffix attention,
 * export/import, the dequantising export, page copies and session files; the fused
 * append + attention entry points store q8 rows only (MIIKV_KV_Q8_Q8,
 * MIIKV_EUNSUPPORTED otherwise). */
enum { MIIKV_KV_FP16_FP16 = 0, MIIKV_KV_Q8_FP16 = 1, MIIKV_KV_FP16_Q8 = 2, MIIKV_KV_Q8_Q8 = 3 };

enum { MIIKV_DTYPE_F16 = 0, MIIKV_DTYPE_F32 = 1 };

/* Non-owning view of one attention layer's KV cache.
 * Replaces AttentionKvCacheView (include/miinfer/prefill_v2/kv_cache.hpp:24-46),
 * adding the block table for paged sequences. */
typedef struct miikv_view {
    int8_t* k_codes;
    uint16_t* k_scales; /* fp16 bits */
    int8_t* v_codes;
    uint16_t* v_scales; /* fp16 bits */
    uint32_t layout;      /* MIIKV_LAYOUT_* */
    uint32_t quant_mode;  /* MIIKV_KV_* */
    uint32_t kv_heads;
    uint32_t head_dim;    /* 128 or 256 */
    uint32_t page_tokens; /* multiple of 64; CONTIGUOUS: the capacity */
    uint32_t num_pages;   /* CONTIGUOUS: 1 */
    const int32_t* block_table; /* PAGED: device [batch][table_stride]; CONTIGUOUS: NULL */
    uint32_t table_stride;      /* PAGED: entries per sequence row */
    uint32_t reserved;
} miikv_view;

/* Mirrors DeviceDecodeState (include/miinfer/qwen3_gpu_primitives.hpp:30-37). */
typedef struct __attribute__((aligned(64))) miikv_decode_state {
    uint32_t current_token;
    uint32_t position; /* position of the token being decoded; context = position + 1 */
    uint32_t generated;
    uint32_t stop;
    uint32_t max_generated;
    uint32_t pad[11];
} miikv_decode_state;

/* Mirrors DevicePrefillState (include/miinfer/qwen3_gpu_primitives.hpp:39-45). */
typedef struct __attribute__((aligned(64))) miikv_prefill_state {
    uint32_t base_position;
    uint32_t token_count;
    uint32_t total_length;
    uint32_t kv_capacity;
    uint32_t pad[12];
} miikv_prefill_state;

/* Advance a device decode state after one step, on the device so that a
 * captured decode graph replays without host work: token_output[generated] =
 * current_token (if token_output != NULL and generated < capacity); stop |=
 * current_token in stop_tokens (host array, at most 8; the reference's
 * Qwen3.5 stop tokens are 151643 and 151645) or generated + 1 >=
 * max_generated; position += 1; generated += 1.
 * Replaces launch_qwen35_decode_state_advance
 * (include/miinfer/qwen3_gpu_primitives.hpp:1248; kernel
 * gfx906/kernels/qwen3_primitives.hip:4417-4429). */
miikv_status miikv_decode_state_advance(miikv_decode_state* state, uint32_t* token_output, uint32_t capacity,
                                        const uint32_t* stop_tokens, uint32_t stop_count, void* stream);

/* A generic device-to-device copy segment for miikv_copy_segments. */
typedef struct miikv_segment {
    void* dst;
    const void* src;
    uint64_t bytes;
} miikv_segment;

/* ---- library ------------------------------------------------------------- */

uint32_t miikv_abi_version(void);
const char* miikv_status_string(miikv_status status);

/* Bytes of each plane for a view's geometry (codes and scales, per K or V). */
miikv_status miikv_plane_bytes(const miikv_view* view, uint64_t* code_bytes, uint64_t* scale_bytes);

/* ---- q8_0 append --------------------------------------------------------- */

/* Quantize `token_count` fp16 K and V rows (layout [token][kv_head][head_dim])
 * into the cache of sequence `seq` at positions base_position .. +token_count-1.
 * If prefill_state is non-NULL, base_position/token_count are read from it on
 * the device (token_count must then be an upper bound; rows beyond the device
 * value are skipped); else if decode_state is non-NULL, one row is stored at
 * decode_state->position.
 * Replaces launch_qwen35_decoupled_k_norm_rope_kv_store_batch_quant
 * (include/miinfer/qwen3_gpu_primitives.hpp:695-717) for pre-normalised fp16
 * rows; the per-row absmax/127 rule (gfx906/kernels/qwen3_primitives.hip:
 * 7285-7322) is applied per 32-value block. */
miikv_status miikv_append_f16(const miikv_view* view, const uint16_t* k, const uint16_t* v,
                              uint32_t token_count, uint32_t base_position, uint32_t seq,
                              const miikv_prefill_state* prefill_state,
                              const miikv_decode_state* decode_state, void* stream);

/* fp32 K/V rows (layout [token][kv_head][head_dim]) into the cache, as
 * miikv_append_f16.  With k_norm_weight != NULL (device fp32 [head_dim],
 * head_dim >= 64) each K row first gets the reference's prologue: RMSNorm
 * x * rsqrt(mean(x^2) + epsilon) * w, then RoPE on dims 0..63 (pairs i, i+32,
 * angle position * theta^(-2i/64)) at its absolute position.  V is stored as
 * given.  This is the drop-in for
 * launch_qwen35_decoupled_k_norm_rope_kv_store_batch_quant
 * (include/miinfer/qwen3_gpu_primitives.hpp:695-717; kernel
 * gfx906/kernels/qwen3_primitives.hip:7213-7365, prologue :7257-7281 and
 * :622-659), with one scale per 32-value block and any head_dim multiple of 32. */
miikv_status miikv_append_f32(const miikv_view* view, const float* k, const float* v,
                              const float* k_norm_weight, uint32_t token_count, uint32_t base_position,
                              uint32_t seq, float theta, float epsilon,
                              const miikv_prefill_state* prefill_state,
                              const miikv_decode_state* decode_state, void* stream);

/* Batched decode append: one fp16 K/V row per sequence (layout [batch][kv_head]
 * [head_dim]); sequence b's row goes to position d_positions[b] (device array).
 * No reference counterpart for batching: the reference decodes one sequence
 * (qwen3_primitives.hip:7239-7241); each row follows the same rule. */
miikv_status miikv_append_batch_f16(const miikv_view* view, const uint16_t* k, const uint16_t* v,
                                    uint32_t batch, const uint32_t* d_positions, void* stream);

/* ---- split-K GQA decode attention ---------------------------------------- */

/* Workspace bytes needed by miikv_decode_attn for `batch` sequences of at most
 * `max_context` tokens (per-split partial softmax records); 0 for an invalid
 * geometry or one decode does not serve (more than 16 query heads per kv head,
 * for which miikv_decode_attn returns MIIKV_EUNSUPPORTED).  Its contents need
 * no initialisation; miikv_workspace_init zero-fills a buffer with a kernel
 * (no memset node), e.g. for reproducible dumps. */
uint64_t miikv_decode_workspace_bytes(const miikv_view* view, uint32_t q_heads, uint32_t batch,
                                      uint32_t max_context);
miikv_status miikv_workspace_init(void* workspace, uint64_t bytes, void* stream);

/* Single-token GQA attention for `batch` sequences over the q8_0 cache.
 *   q       device [batch][q_heads][head_dim], fp16 or fp32 (q_dtype)
 *   context length of sequence b: d_lengths[b] if d_lengths != NULL, else
 *           decode_state->position + 1 (batch must be 1)
 *   max_context  host upper bound on every context length (sizes the grid)
 *   out     device [batch][q_heads][head_dim] fp32 (nullable)
 *   gate    device [batch][q_heads][head_dim] fp32 (nullable); gated_out =
 *           out * sigmoid(gate) (nullable).  At least one output is required.
 * Replaces launch_qwen35_tiled_online_attention_quant_dynamic
 * (include/miinfer/qwen3_gpu_primitives.hpp:719-741; kernels
 * gfx906/kernels/qwen3_primitives.hip:7371-7548 and 2295-2385) with an explicit
 * workspace instead of module-static split scratch. */
miikv_status miikv_decode_attn(const miikv_view* view, const void* q, uint32_t q_dtype,
                               uint32_t q_heads, float scale, uint32_t batch,
                               const uint32_t* d_lengths, const miikv_decode_state* decode_state,
                               uint32_t max_context, float* out, const float* gate,
                               float* gated_out, void* workspace, uint64_t workspace_bytes,
                               void* stream);

/* miikv_decode_attn plus the reference's Q8_1 output epilogue: with gate set,
 * gated_q8_1 (nullable, device, 36-byte blocks {fp16 d, fp16 s, int8 qs[32]},
 * [batch][q_heads][head_dim/32]) receives gated_out quantized per 32 values:
 * d = amax/127, qs = clamp(roundf(x/d), -127, 127), s = sum(qs)*d — the
 * `gated_output_q8` argument of launch_qwen35_tiled_online_attention_quant_dynamic
 * (include/miinfer/qwen3_gpu_primitives.hpp:719-741; emit
 * gfx906/kernels/qwen3_primitives.hip:2354-2384; block
 * include/miinfer/q4_q8_gemv.hpp:23-27), consumed by the O-projection GEMV.
 * gated_out may then be NULL. */
miikv_status miikv_decode_attn_q8_1(const miikv_view* view, const void* q, uint32_t q_dtype, uint32_t q_heads,
                                    float scale, uint32_t batch, const uint32_t* d_lengths,
                                    const miikv_decode_state* decode_state, uint32_t max_context, float* out,
                                    const float* gate, float* gated_out, void* gated_q8_1, void* workspace,
                                    uint64_t workspace_bytes, void* stream);

/* Fused append + decode: stores the new fp16 K/V row of each sequence
 * (k_new, v_new device [batch][kv_heads][head_dim]) at position L-1 of that
 * sequence, where L is the context length including it (d_lengths[b] or
 * decode_state->position + 1), with the append rule, and attends over all L
 * keys — one launch pair instead of the reference's store kernel followed by
 * attention (attention_layer.cpp:599-632).  Cache bytes and results equal
 * miikv_append_f16 followed by miikv_decode_attn_q8_1. */
miikv_status miikv_decode_append_attn(const miikv_view* view, const uint16_t* k_new, const uint16_t* v_new,
                                      const void* q, uint32_t q_dtype, uint32_t q_heads, float scale,
                                      uint32_t batch, const uint32_t* d_lengths,
                                      const miikv_decode_state* decode_state, uint32_t max_context, float* out,
                                      const float* gate, float* gated_out, void* gated_q8_1, void* workspace,
                                      uint64_t workspace_bytes, void* stream);

/* The reference's decode step in one launch pair with its own store arguments:
 * k_new / v_new are fp32 rows [batch][kv_heads][head_dim] as the reference store
 * kernel takes them; with k_norm_weight set, K first gets the reference's prologue
 * (RMSNorm * weight with epsilon, RoPE on dims 0..63 with theta at the row's
 * position L-1) before the q8 rule.  Replaces
 * launch_qwen35_decoupled_k_norm_rope_kv_store_batch_quant followed by
 * launch_qwen35_tiled_online_attention_quant_dynamic (attention_layer.cpp:599-632;
 * include/miinfer/qwen3_gpu_primitives.hpp:695-741).  Cache bytes equal
 * miikv_append_f32 with the same arguments; outputs as miikv_decode_append_attn. */
miikv_status miikv_decode_append_attn_f32(const miikv_view* view, const float* k_new, const float* v_new,
                                          const float* k_norm_weight, float theta, float epsilon, const void* q,
                                          uint32_t q_dtype, uint32_t q_heads, float scale, uint32_t batch,
                                          const uint32_t* d_lengths, const miikv_decode_state* decode_state,
                                          uint32_t max_context, float* out, const float* gate, float* gated_out,
                                          void* gated_q8_1, void* workspace, uint64_t workspace_bytes,
                                          void* stream);

/* miikv_decode_append_attn without the workspace arguments, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The split records go
 * to a fixed device array inside the library, one per GPU, of
 * miikv_decode_scratch_max_bytes() bytes (16 MiB: one 32q/8kv/D128 sequence at
 * any context needs ~1.1 MB, 16 sequences of 24q/4kv/D256 up to 64k ~13 MB); a
 * geometry whose
 * miikv_decode_workspace_bytes() exceeds it returns MIIKV_EWORKSPACE.  Nothing is
 * allocated (the array's address is looked up, and one event made, once per device
 * at the first call).  All calls on one GPU share that array, so the library orders
 * them: one host lock covers each call's enqueue, and a call on another stream than
 * the previous call's waits for an event recorded after that call's kernels.  Inside
 * a stream capture that wait and record are left out (the graph's order applies):
 * replays of captured graphs that overlap on one GPU (several streams at once) race
 * on the array and must be serialised by the caller. */
uint64_t miikv_decode_scratch_max_bytes(void);
miikv_status miikv_decode_append_attn_noalloc(const miikv_view* view, const uint16_t* k_new,
                                              const uint16_t* v_new, const void* q, uint32_t q_dtype,
                                              uint32_t q_heads, float scale, uint32_t batch,
                                              const uint32_t* d_lengths, const miikv_decode_state* decode_state,
                                              uint32_t max_context, float* out, const float* gate,
                                              float* gated_out, void* gated_q8_1, void* stream);

/* ---- suffix (multi-token) attention over a cached prefix ----------------- */

/* Causal attention of a token_count-token suffix whose rows already sit in the
 * cache at positions base_position .. base_position+token_count-1 (append them
 * first); token t attends to positions [0, base_position + t].
 *   q    device [token_count][q_heads][head_dim], fp16 or fp32 (fp32 is rounded
 *        to fp16 for the MFMA)
 *   out / gated_out  device [token_count][q_heads][head_dim] fp32; gated_out =
 *        out * sigmoid(gate).  At least one output is required.
 * If prefill_state is non-NULL, base_position and token_count come from it on
 * the device (token_count is then a host upper bound).
 * A short suffix runs as a batch of decodes over the sequence (up to 16 / (q_heads
 * / kv_heads) tokens share one pass over the context; at most 12 such passes for
 * caches of at most 16384 positions, 6 above); longer ones run on MFMA over fp16
 * tiles expanded into the workspace.  miikv_suffix_workspace_bytes() covers both; a smaller workspace
 * that holds the tiles runs the MFMA path with one split.
 * Accuracy of the MFMA path: its operands are fp16 (the query rounded once, each key
 * and value element code * scale rounded once, the probabilities rounded once), which
 * keeps outputs within max-abs 2e-3 and relative 1e-2 of fp32 attention over the same
 * cache when the logits (scale * q.k) have a standard deviation up to 2, and within
 * max-abs 1.5e-2 and relative 2e-3 up to 6.  Sharper attention that needs the
 * reference's fp32 products takes MIIKV_SUFFIX_EXACT (miikv_suffix_attn_ex), within
 * max-abs 2e-3 and relative 1e-2 there.
 * Replaces launch_qwen35_splitk_suffix_attention_quant
 * (include/miinfer/qwen3_gpu_primitives.hpp:670-693; kernels
 * gfx906/kernels/qwen3_primitives.hip:6789-7207, 6637-6725). */
uint64_t miikv_suffix_workspace_bytes(const miikv_view* view, uint32_t q_heads, uint32_t token_count);
miikv_status miikv_suffix_attn(const miikv_view* view, const void* q, uint32_t q_dtype,
                               uint32_t q_heads, float scale, uint32_t token_count,
                               uint32_t base_position, uint32_t seq,
                               const miikv_prefill_state* prefill_state, float* out,
                               const float* gate, float* gated_out, void* workspace,
                               uint64_t workspace_bytes, void* stream);

/* Fused append + suffix attention: quantises the suffix's own fp16 K/V rows
 * (k_new, v_new device [token_count][kv_heads][head_dim]) with the append rule,
 * stores them at positions base_position + t (or the prefill state's), and
 * attends as miikv_suffix_attn, in one pass over the context instead of the
 * reference's store launch followed by attention (attention_layer.cpp:297-343);
 * a short suffix (see miikv_suffix_attn) is stored first, then attended.
 * Cache bytes and results equal miikv_append_f16 followed by miikv_suffix_attn. */
miikv_status miikv_suffix_append_attn(const miikv_view* view, const uint16_t* k_new, const uint16_t* v_new,
                                      const void* q, uint32_t q_dtype, uint32_t q_heads, float scale,
                                      uint32_t token_count, uint32_t base_position, uint32_t seq,
                                      const miikv_prefill_state* prefill_state, float* out,
                                      const float* gate, float* gated_out, void* workspace,
                                      uint64_t workspace_bytes, void* stream);

/* Suffix attention with flags; k_new / v_new optional (both set: as
 * miikv_suffix_append_attn, both NULL: as miikv_suffix_attn).
 * MIIKV_SUFFIX_TILES_CURRENT (chunked prefill, the reference's 512-token tiles over
 * a growing prefix, attention_layer.cpp:297-343): the workspace keeps the fp16
 * tiles of this sequence's context between calls, at a fixed per-head stride of
 * the cache capacity, and the caller asserts that the tiles of every key below the
 * base position (the prefill state's, when given) were expanded by earlier calls
 * with this flag, this workspace and this sequence, and that those cache rows are
 * unchanged since.  Each call then expands only the steps from the one holding the
 * base position on (instead of the whole context) and leaves its own steps current
 * for the next call, also when a short suffix runs as decodes.  One workspace per
 * (layer, sequence); a workspace of miikv_suffix_workspace_bytes() bytes suffices.
 * The first call of a sequence (base position 0) needs no earlier call.
 * MIIKV_SUFFIX_EXACT: the reference's fp32 products (qwen3_primitives.hip:6789-7207)
 * to the decode path's precision, where the MFMA path takes the query and the
 * dequantised keys as fp16: an fp32 query's low half is kept and the key block scales
 * are applied in fp32.  A long suffix over q8 planes runs on exact-product MFMA
 * kernels (key codes as exact fp16, one MFMA per 32-value block with its scale in
 * fp32, a second one for the query's low half; about 2.2x the MFMA path at config 4);
 * short suffixes, the other quant modes and chunked prefill (TILES_CURRENT) run every
 * token as a decode (batches of decodes over the sequence).  Needs q_heads / kv_heads
 * <= 16 (else MIIKV_EUNSUPPORTED) and a workspace of
 * miikv_suffix_workspace_bytes_ex(view, q_heads, token_count, flags) bytes (else
 * MIIKV_EWORKSPACE; it never falls back to the fp16 MFMA path). */
#define MIIKV_SUFFIX_TILES_CURRENT 1u
#define MIIKV_SUFFIX_EXACT 2u
/* Workspace of miikv_suffix_attn_ex with `flags`: miikv_suffix_workspace_bytes(),
 * or more with MIIKV_SUFFIX_EXACT; 0 for invalid arguments or an unsupported
 * geometry. */
uint64_t miikv_suffix_workspace_bytes_ex(const miikv_view* view, uint32_t q_heads, uint32_t token_count,
                                         uint32_t flags);
miikv_status miikv_suffix_attn_ex(const miikv_view* view, const uint16_t* k_new, const uint16_t* v_new,
                                  const void* q, uint32_t q_dtype, uint32_t q_heads, float scale,
                                  uint32_t token_count, uint32_t base_position, uint32_t seq,
                                  const miikv_prefill_state* prefill_state, uint32_t flags, float* out,
                                  const float* gate, float* gated_out, void* workspace,
                                  uint64_t workspace_bytes, void* stream);

/* ---- export / import ----------------------------------------------------- */

/* Copy tokens [t0, t0+count) of sequence `seq` out of the tiled cache into
 * canonical row-major buffers: codes [kv_heads][count][head_dim] and scales
 * [kv_heads][count][head_dim/32] (any pointer may be NULL to skip that plane).
 * This is the device half of download_raw (src/prefill_v2/kv_cache.cpp:227-297). */
miikv_status miikv_export_canonical(const miikv_view* view, uint32_t seq, uint32_t t0,
                                    uint32_t count, int8_t* k_codes, uint16_t* k_scales,
                                    int8_t* v_codes, uint16_t* v_scales, void* stream);

/* Dequantised rows of tokens [t0, t0+count) of sequence `seq`: k_out / v_out
 * device fp32 [kv_heads][count][head_dim] (16-byte aligned; either may be NULL),
 * value = float(code) * float(scale).  The device half of the q8 branch of
 * AttentionLayerKvCacheStorage::download_key / download_value
 * (src/prefill_v2/kv_cache.cpp:132-212), for debug dumps and float read-back. */
miikv_status miikv_export_dequant(const miikv_view* view, uint32_t seq, uint32_t t0, uint32_t count,
                                  float* k_out, float* v_out, void* stream);

/* Inverse of miikv_export_canonical (device half of upload_raw,
 * src/prefill_v2/kv_cache.cpp:299-369). */
miikv_status miikv_import_canonical(const miikv_view* view, uint32_t seq, uint32_t t0,
                                    uint32_t count, const int8_t* k_codes,
                                    const uint16_t* k_scales, const int8_t* v_codes,
                                    const uint16_t* v_scales, void* stream);

/* ---- prefix-state reuse --------------------------------------------------- */

/* Copy n physical pages (all four planes) src_pages[i] -> dst_pages[i]
 * (device int32 arrays), byte for byte.  Block-granular KV copy used by
 * copy-on-write forks.  No reference counterpart: the reference keeps a single
 * contiguous cache in place (src/prefill_v2/model.cpp:752-846). */
miikv_status miikv_copy_pages(const miikv_view* view, const int32_t* d_src_pages,
                              const int32_t* d_dst_pages, uint32_t n, void* stream);

/* Execute n device-to-device copies described by a DEVICE array of segments in
 * one launch.  Replaces the 2*48 hipMemcpyAsync calls of
 * GdnCheckpointStorage::capture/restore (src/prefill_v2/reusable_context.cpp:65-128). */
miikv_status miikv_copy_segments(const miikv_segment* d_segments, uint32_t n, void* stream);

/* Clone `bytes` of src into each of n destinations (device array of pointers):
 * the recurrent-state clone of forked sessions.  bytes must be a multiple of 16
 * and every pointer 16-byte aligned. */
miikv_status miikv_clone_state(void* const* d_dsts, const void* src, uint64_t bytes, uint32_t n,
                               void* stream);

/* ---- prefix reuse: host-side policy (no device work) ---------------------- */

/* Page pool with reference counts for paged caches.  Forked sequences share full
 * pages; a partial last page is copied (copy-on-write) so the child can append.
 * No reference counterpart: the reference keeps one contiguous cache per layer
 * and reuses a prefix in place (src/prefill_v2/model.cpp:752-846). */
typedef struct miikv_pool miikv_pool;
miikv_pool* miikv_pool_create(uint32_t num_pages);
void miikv_pool_destroy(miikv_pool* pool);
int32_t miikv_pool_alloc(miikv_pool* pool);                 /* -1 when exhausted */
miikv_status miikv_pool_ref(miikv_pool* pool, int32_t page);
miikv_status miikv_pool_unref(miikv_pool* pool, int32_t page); /* frees at zero */
uint32_t miikv_pool_refcount(const miikv_pool* pool, int32_t page);
uint32_t miikv_pool_free_pages(const miikv_pool* pool);
/* Fork a sequence of `length` tokens: child_row[0..pages) shares the parent's
 * full pages (reference +1); a partial last page gets a fresh page and one
 * (copy_src, copy_dst) pair to run with miikv_copy_pages.  parent_row and
 * child_row each hold row_capacity entries (MIIKV_EINVAL if the sequence needs
 * more pages). */
miikv_status miikv_pool_fork(miikv_pool* pool, const int32_t* parent_row, uint32_t row_capacity,
                             uint32_t length, uint32_t page_tokens, int32_t* child_row,
                             int32_t* copy_src, int32_t* copy_dst, uint32_t* n_copies);
/* n forks of one parent in one call (child i's row at child_rows + i*row_stride,
 * row_stride >= pages of `length`); copy_src / copy_dst (capacity n) receive the
 * copy-on-write page pairs and *n_copies their count; *n_done forks completed
 * (all on success; fewer with MIIKV_EINVAL on pool exhaustion). */
miikv_status miikv_pool_fork_n(miikv_pool* pool, const int32_t* parent_row, uint32_t length, uint32_t page_tokens,
                               uint32_t n, int32_t* child_rows, uint32_t row_stride, int32_t* copy_src,
                               int32_t* copy_dst, uint32_t* n_copies, uint32_t* n_done);
/* Before appending at `position` (the sequence's current length): allocate a
 * fresh page at a page boundary, or copy a shared page (copy-on-write).  Row
 * entries not backing a token yet must be -1; an entry that already holds a page
 * (a repeated call for the same position) keeps it, copied only if shared. */
miikv_status miikv_pool_prepare_append(miikv_pool* pool, int32_t* row, uint32_t row_capacity,
                                       uint32_t position, uint32_t page_tokens,
                                       int32_t* copy_src, int32_t* copy_dst, uint32_t* n_copies);
/* Drop one reference on each page backing `length` tokens of `row`, and set
 * those entries to -1 (a released row starts over as an empty row). */
miikv_status miikv_pool_release(miikv_pool* pool, int32_t* row, uint32_t length,
                                uint32_t page_tokens);

/* Prefix fingerprint and match policy.  Restates ReusableContext
 * (include/miinfer/prefill_v2/reusable_context.hpp:17-129,
 * src/prefill_v2/reusable_context.cpp:130-207); results keep its enum order. */
#define MIIKV_STATE_LAYOUT_VERSION 20260925u
enum {
    MIIKV_MATCH_EXACT = 0,
    MIIKV_MATCH_PREFIX_MISMATCH = 1,
    MIIKV_MATCH_MODEL_MISMATCH = 2,
    MIIKV_MATCH_QUANTIZATION_MISMATCH = 3,
    MIIKV_MATCH_EMPTY_CACHE = 4,
    MIIKV_MATCH_PROMPT_SHORTER = 5,
    MIIKV_MATCH_VERSION_MISMATCH = 6,
};
typedef struct miikv_prefix_ctx miikv_prefix_ctx;
uint64_t miikv_token_hash(const uint32_t* tokens, size_t count); /* FNV-1a 64 */
miikv_prefix_ctx* miikv_prefix_create(const char* model_id, const char* quantization);
void miikv_prefix_destroy(miikv_prefix_ctx* ctx);
miikv_status miikv_prefix_save(miikv_prefix_ctx* ctx, const uint32_t* tokens, size_t count);
int miikv_prefix_check(const miikv_prefix_ctx* ctx, const uint32_t* prompt, size_t count,
                       const char* model_id, const char* quantization);
void miikv_prefix_clear(miikv_prefix_ctx* ctx);
uint32_t miikv_prefix_length(const miikv_prefix_ctx* ctx);
uint64_t miikv_prefix_hash(const miikv_prefix_ctx* ctx);
void miikv_prefix_set_layout_version(miikv_prefix_ctx* ctx, uint32_t version);

/* Registry of several saved prefixes over one page pool (the reference keeps a
 * single ReusableContext slot: src/prefill_v2/reusable_context.cpp:130-207, used
 * by src/prefill_v2/model.cpp:752-871).  An entry holds the fingerprint (tokens,
 * FNV-1a hash, layout version; model and quantization are the registry's) and
 * one pool reference on each page of its row, so its KV pages outlive the
 * session that wrote them.  `tag` is the caller's handle for the entry's
 * recurrent-state checkpoint (device memory the caller owns).
 *   save:    register tokens[0..count) held by row[0..pages); the same tokens
 *            again refresh the existing entry; MIIKV_EWORKSPACE when full
 *            (evict first).
 *   lookup:  the longest entry whose prefix matches under check_match's rule
 *            (reusable_context.cpp:155-185; strict != 0 also requires a shorter
 *            prefix than the prompt, as generate() does); without a match the
 *            verdict for the most recently used entry, EMPTY_CACHE when empty.
 *   fork:    a session row from an entry (full pages shared, partial last page
 *            copied: one (copy_src, copy_dst) pair for miikv_copy_pages).
 *   release / evict_lru: drop an entry (its page references go back to the
 *            pool); report its tag so the caller frees the checkpoint. */
typedef struct miikv_registry miikv_registry;
miikv_registry* miikv_registry_create(miikv_pool* pool, uint32_t page_tokens, uint32_t max_entries,
                                      const char* model_id, const char* quantization);
void miikv_registry_destroy(miikv_registry* reg);
uint32_t miikv_registry_count(const miikv_registry* reg);
miikv_status miikv_registry_save(miikv_registry* reg, const uint32_t* tokens, uint32_t count, const int32_t* row,
                                 uint32_t row_capacity, uint64_t tag, uint32_t* entry_id_out);
int miikv_registry_lookup(const miikv_registry* reg, const uint32_t* prompt, uint32_t count,
                          const char* model_id, const char* quantization, uint32_t strict,
                          uint32_t* entry_id_out, uint32_t* prefix_length_out);
miikv_status miikv_registry_fork(miikv_registry* reg, uint32_t entry_id, int32_t* child_row,
                                 uint32_t row_capacity, int32_t* copy_src, int32_t* copy_dst,
                                 uint32_t* n_copies);
miikv_status miikv_registry_release(miikv_registry* reg, uint32_t entry_id, uint64_t* tag_out);
miikv_status miikv_registry_evict_lru(miikv_registry* reg, uint32_t* entry_id_out, uint64_t* tag_out);
miikv_status miikv_registry_info(const miikv_registry* reg, uint32_t entry_id, uint32_t* length,
                                 uint64_t* token_hash, uint64_t* tag, int32_t* pages, uint32_t pages_cap);
miikv_status miikv_registry_set_layout_version(miikv_registry* reg, uint32_t entry_id, uint32_t version);

/* ---- persistent session file (.miinfer) ----------------------------------- */

/* On-disk session state, the reference's PersistentSessionHeader
 * (include/miinfer/prefill_v2/persistent_session.hpp:18-34): packed, 157 bytes,
 * magic "MISS", version 20260928, followed by prefix_length u32 tokens, the
 * recurrent state bytes (per GDN layer: state then conv history, in segment
 * order) and the KV bytes (per attention layer the raw compact form of
 * src/prefill_v2/kv_cache.cpp:227-297: for each kv head its K part -- fp16 rows
 * [P][D], or q8 codes [P][D] then scales -- then the same for V).  kv_quant_mode
 * is the cache's mode (persistent_session.cpp:54 writes the model's mode): an
 * FP16_FP16 cache is written as the reference's mode 0 (kv_cache.hpp:16-21), byte
 * for byte its raw format; a cache with a q8 plane holds one fp16 scale per
 * 32-value block ([P][D/32] per head, where the reference's modes 1..3 hold one per
 * row), so it gets a value of its own: MIIKV_SESSION_KV_Q8_0_32 (both planes q8),
 * ..._Q8_0_32_FP16 (q8 K, fp16 V), ..._FP16_Q8_0_32 (fp16 K, q8 V).  The
 * reference's per-row modes 1..3 are not produced here and are rejected on load. */
#define MIIKV_SESSION_VERSION 20260928u
#define MIIKV_SESSION_KV_FP16_FP16 0u
#define MIIKV_SESSION_KV_Q8_0_32 4u
#define MIIKV_SESSION_KV_Q8_0_32_FP16 5u
#define MIIKV_SESSION_KV_FP16_Q8_0_32 6u
#pragma pack(push, 1)
typedef struct miikv_session_header {
    char magic[4];
    uint32_t version;
    char model_id[64];
    char quantization[32];
    uint32_t prefix_length;
    uint64_t token_hash;
    uint32_t gdn_layers;
    uint64_t gdn_state_bytes;
    uint32_t gqa_layers;
    uint8_t kv_quant_mode;
    uint64_t kv_bytes;
    uint64_t tokens_bytes;
    uint64_t created_timestamp;
} miikv_session_header;
#pragma pack(pop)

/* The session-file kv_quant_mode written for a view quant mode (MIIKV_KV_*);
 * 0xff for an unknown mode. */
uint32_t miikv_session_kv_mode(uint32_t view_quant_mode);

/* "sess_<16 hex digits of token_hash>_p<prefix_length>.miinfer" into out
 * (persistent_session.cpp:27-32).  Returns MIIKV_EINVAL if out_cap is short. */
miikv_status miikv_session_filename(uint64_t token_hash, uint32_t prefix_length, char* out, size_t out_cap);

/* Save a session (persistent_session.cpp:34-136): the first prefix_length
 * tokens of sequence `seq` of every attention layer view, and the recurrent
 * state given as gdn_segment_count device segments (state, conv, state, conv,
 * ...; gdn_layers = count / 2).  Written to "<path>.tmp" and renamed.  Device
 * reads are ordered on `stream`; the call returns after the file is written.
 * Allocates a device staging buffer of one layer's KV bytes for the call. */
miikv_status miikv_session_save(const char* path, const char* model_id, const char* quantization,
                                const uint32_t* tokens, uint32_t prefix_length, const miikv_view* kv_layers,
                                uint32_t kv_layer_count, uint32_t seq, void* const* gdn_segments,
                                const uint64_t* gdn_segment_bytes, uint32_t gdn_segment_count, void* stream);

/* Read and validate the header (magic, version) and, if tokens_out is not NULL,
 * up to tokens_cap prefix tokens (persistent_session.cpp:138-161).  Returns 1
 * on success, 0 otherwise. */
int miikv_session_inspect(const char* path, miikv_session_header* out, uint32_t* tokens_out, uint32_t tokens_cap);

/* Load a session (persistent_session.cpp:163-258): checks magic, version, model
 * id, quantization, layer counts, kv_quant_mode, sizes and the token hash, then
 * writes the KV of every layer (positions 0..P-1 of sequence `seq`) and the
 * recurrent segments.  *prefix_length_out = P; the tokens go to tokens_out
 * (tokens_cap >= P).  Returns 1 on success, 0 if the file does not match (no
 * device memory is written then), or a negative HIP status. */
int miikv_session_load(const char* path, const char* model_id, const char* quantization,
                       const miikv_view* kv_layers, uint32_t kv_layer_count, uint32_t seq,
                       void* const* gdn_segments, const uint64_t* gdn_segment_bytes, uint32_t gdn_segment_count,
                       uint32_t* tokens_out, uint32_t tokens_cap, uint32_t* prefix_length_out, void* stream);

/* The longest saved prefix of `prompt` among the .miinfer files of session_dir
 * for this model and quantization (persistent_session.cpp:260-320): returns 1
 * and fills path_out / *prefix_length_out, or 0 if none matches. */
int miikv_session_find(const char* session_dir, const char* model_id, const char* quantization,
                       const uint32_t* prompt, size_t prompt_len, char* path_out, size_t path_cap,
                       uint32_t* prefix_length_out);

/* ---- measurement probe --------------------------------------------------- */

/* Read `bytes` from src once with 16-byte nontemporal loads over `blocks`
 * workgroups of 256 threads (bytes must be a multiple of 16*blocks), writing
 * one fold word per workgroup to sink[blocks].  A streaming-read ceiling for
 * the roofline of the decode kernels; no reference counterpart. */
miikv_status miikv_stream_read(const void* src, uint64_t bytes, uint32_t* sink, uint32_t blocks,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MIIKV_H */
