// Definitions of the suffix-attention kernels (miikv_suffix.hip): launch
// constants, argument blocks, the split-record layout and small device helpers.
#pragma once
#include "miikv_common.hpp"

namespace miikv {

#ifndef MIIKV_SUFFIX_WAVES
#define MIIKV_SUFFIX_WAVES 8
#endif
constexpr uint32_t kSufWaves = MIIKV_SUFFIX_WAVES;
constexpr uint32_t kSufRows = 32 * kSufWaves;  // query rows per workgroup
constexpr uint32_t kSufStep = 32;              // keys per step
constexpr float kLog2eS = 1.4426950408889634f;
constexpr float kSlackS = 6.0f;        // lazy-rescale threshold (log2 units): p <= 64
// Resident workgroups of suffix_kernel on the chip: 256 CUs, each holding 8 waves
// (two per SIMD at <= 256 VGPRs) and its LDS tile buffers (4 x 32 KiB at D = 256).
constexpr uint32_t kSufSlots = 256 * (8 / kSufWaves);
constexpr uint32_t kSufMaxSplits = 64;
// Suffixes of at most this many decode row sets (tokens / tokens packed per row set)
// run as a batch of decodes (miikv_decode.hip): caches of more than 16384 positions,
// and of at most that many.
constexpr uint32_t kSuffixDecodeMaxRows = 6;
constexpr uint32_t kSuffixDecodeMaxRowsShort = 12;
constexpr uint32_t kSuffixDecodeMaxT = 64;
uint32_t suffix_pack(const miikv_view* view, uint32_t q_heads, uint32_t token_count, bool device_count,
                     uint32_t max_cols = 16);
bool decode_columns_fit(uint32_t G, uint32_t D);  // decode_kernel serves G columns at head_dim D
uint64_t suffix_by_decode_bytes(const miikv_view* view, uint32_t q_heads, uint32_t token_count, uint32_t bound);
miikv_status suffix_by_decode(const miikv_view* view, const void* q, uint32_t q_dtype, uint32_t q_heads, float scale,
                              uint32_t token_count, uint32_t base_position, uint32_t seq,
                              const miikv_prefill_state* prefill_state, uint32_t bound, float* out, const float* gate,
                              float* gated_out, void* workspace, uint64_t workspace_bytes, void* stream);

// fp16 halves of one expanded step: K fragments [D/16][64 lanes][8], then
// V fragments [D/32][2 key halves][64 lanes][8].
__host__ __device__ constexpr uint32_t tile_halves(uint32_t D) { return 2 * D * kSufStep; }

struct ExpandArgs {
    Geo g;
    uint32_t seq;
    uint32_t key_count;  // host: P + T; with a device state: the capacity bound
    const miikv_prefill_state* ps;
    uint32_t steps;      // steps per kv head in the tile area
    _Float16* tiles;
    // Fused append (k_new set): the suffix's fp16 rows [token_count][kv_heads][D],
    // quantised and stored at positions base_position + t (or the prefill state's).
    const uint16_t* k_new;
    const uint16_t* v_new;
    uint32_t token_count;
    uint32_t base_position;
    // Incremental tiles: grid x covers steps step0 + (gridDim.x - 1 - blockIdx.x); with
    // `current` set the steps wholly below the base position (the prefill state's, on
    // the device) are already expanded in the tile area and are skipped.
    uint32_t step0;
    uint32_t current;
};

struct SuffixArgs {
    Geo g;
    const void* q;
    uint32_t q_f32;
    uint32_t q_heads;
    uint32_t group;
    float scale_log2;
    uint32_t token_count;  // host upper bound
    uint32_t base_position;
    const miikv_prefill_state* ps;
    uint32_t split_keys;   // keys per split (multiple of kSufStep)
    uint32_t splits;
    uint32_t row_blocks;   // workgroups per (kv head, split) group
    uint32_t steps;        // steps per kv head in the tile area
    const _Float16* tiles;
    void* part;            // partial records when splits > 1
    float* out;
    const float* gate;
    float* gated_out;
    uint32_t rows_together;  // suffix_kernel order: (kv head, row block, split) when set
};

// Partial records of split-K, laid out so that a wave's 32 rows write one
// contiguous block: O / l in fp16 [split][kv head][row][D] (row = t*G + g, rows
// counted up to the host token bound), then (m, l) fp32 pairs [split][kv head][row].
// The split's output is stored normalised (a convex combination of V rows, so
// fp16 holds it to the same relative precision as the fp16 V tiles it came from),
// which halves the record traffic of the split kernel and the combine.
struct SuffixCombineArgs {
    uint32_t kv_heads;
    uint32_t q_heads;
    uint32_t group;
    uint32_t token_count;  // host bound
    uint32_t base_position;
    const miikv_prefill_state* ps;
    uint32_t split_keys;
    uint32_t splits;
    const void* part;
    float* out;
    const float* gate;
    float* gated_out;
};

__host__ __device__ inline size_t part_o_halves(uint32_t splits, uint32_t kv_heads, uint32_t rows, uint32_t D) {
    return static_cast<size_t>(splits) * kv_heads * rows * D;
}
// Bytes of one row's record in one split: D fp16 values and an (m, l) pair.
__host__ __device__ constexpr uint32_t part_row_bytes(uint32_t D) { return 2 * D + 8; }

__device__ __forceinline__ float sfx_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float16v mfma_32x32x16(half8 a, half8 b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Wait until at most N vector-memory operations of this wave are outstanding.
template <uint32_t N>
__device__ __forceinline__ void wait_vmem_le() {
    static_assert(N < 64, "vmcnt holds 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
}

}  // namespace miikv
