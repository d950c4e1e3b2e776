// Split-K partial records and their combine, shared by decode and suffix attention.
#pragma once

#include "miikv_common.hpp"

namespace miikv {
namespace {

#ifndef MIIKV_WPW
#define MIIKV_WPW 4
#endif
constexpr uint32_t kWavesPerWg = MIIKV_WPW;

struct SplitArgs {
    Geo g;
    const void* q;
    uint32_t q_heads;
    uint32_t group;  // columns per (row set, kv head), <= 16: pack tokens x query heads per kv head
    // Tokens per row set (1: decode).  A short suffix packs `pack` consecutive tokens of
    // one sequence into a row set: column c is token pack*b + c / (group / pack), query
    // head h * (group / pack) + c % (group / pack), with context split_length() - (pack -
    // 1 - c / (group / pack)).
    uint32_t pack;
    float scale_log2;
    // Context length of row-set b: (len_ptr ? len_ptr[b * len_stride] : 0) + len_add
    // + b * len_bstep (decode: per-sequence lengths; suffix: base + t + 1).
    const uint32_t* len_ptr;
    uint32_t len_stride;
    uint32_t len_add;
    uint32_t len_bstep;
    const uint32_t* count_ptr;  // if set, row-sets b >= *count_ptr are skipped
    uint32_t max_context;
    uint32_t cpw;         // chunks per wave
    uint32_t max_splits;  // splits per (sequence, kv head)
    uint32_t batch;       // sequences (row-sets)
    uint32_t max_cpw;     // cap of the device-side steps per wave
    // batch > 1: resident workgroups of the split kernel; the steps per wave are
    // then chosen on the device from the lengths (at least cpw), 0: always cpw
    uint32_t slots;
    float* part;          // [batch][kv_heads][max_splits + 1][record]: the splits, then
                          // with the fused append the new token's record at slot nsplit
    float* out;
    const float* gate;
    float* gated_out;
    uint8_t* gated_q8_1;  // nullable: Q8_1 blocks [batch][q_heads][D/32] of gated_out
    const uint16_t* k_new;  // fused append: fp16 rows [batch][kv_heads][D] stored at position L-1
    const uint16_t* v_new;
    // fused append of fp32 rows instead (k_new / v_new then null), with the reference's
    // K prologue when k_norm_weight is set (RMSNorm * weight, RoPE on dims 0..63)
    const float* k_new32;
    const float* v_new32;
    const float* k_norm_weight;
    float rope_step;        // theta^(-2/64), from the host
    float epsilon;
    uint32_t q_f32;         // q dtype (scoring the appended token)
    uint32_t rowset_order;  // row sets of one sequence: XCD-ordered (kv head, split, row set) items
};


__device__ __forceinline__ float exp2_safe(float x) { return exp2f(x); }  // exp2(-inf) == 0

// Floats in one split's partial record: O [G*D], m [G], l [G], padded to 4.
__host__ __device__ __forceinline__ uint32_t record_floats(uint32_t G, uint32_t D) {
    return G * D + ((2 * G + 3) / 4) * 4;
}

__device__ __forceinline__ uint32_t split_length(const SplitArgs& a, uint32_t b) {
    uint32_t L = (a.len_ptr ? a.len_ptr[static_cast<size_t>(b) * a.len_stride] : 0u) + a.len_add + b * a.len_bstep;
    return L > a.max_context ? a.max_context : L;
}

// Steps per wave of a launch.  One sequence: the host's cpw.  A batch: the lengths
// are only known on the device, so every workgroup of both kernels derives the
// same value from them: the smallest cpw (>= the host's, which sized the records)
// for which the work items, at most sum(L_b) * H / (4 waves * 32 * cpw) + count * H,
// fit in one round of `slots` resident workgroups.  Called by every thread of the
// workgroup (barriers inside); the first 256 threads do the sum.
__device__ uint32_t launch_cpw(const SplitArgs& a) {
    if (a.batch == 1 || a.slots == 0) return a.cpw;
    __shared__ unsigned long long s_sum[256];
    const uint32_t tid = threadIdx.x;
    const uint32_t count = a.count_ptr ? min(a.batch, *a.count_ptr) : a.batch;
    unsigned long long sum = 0;
    for (uint32_t bb = tid; bb < count && tid < 256; bb += 256) sum += split_length(a, bb);
    if (tid < 256) s_sum[tid] = sum;
    __syncthreads();
    for (uint32_t off = 128; off > 0; off >>= 1) {
        if (tid < off) s_sum[tid] += s_sum[tid + off];
        __syncthreads();
    }
    const unsigned long long total = s_sum[0] * a.g.kv_heads;
    __syncthreads();  // s_sum is reused by the next call
    const unsigned long long fixed_items = static_cast<unsigned long long>(count) * a.g.kv_heads;
    const unsigned long long room = a.slots > fixed_items ? a.slots - fixed_items : a.slots;
    const unsigned long long per = static_cast<unsigned long long>(kWavesPerWg) * kChunk * room;
    const unsigned long long cpw = (total + per - 1) / per;
    return static_cast<uint32_t>(cpw < a.cpw ? a.cpw : (cpw > a.max_cpw ? a.max_cpw : cpw));
}

// Split count of sequence b at `cpw` steps per wave (0 when L == 0).
__device__ __forceinline__ uint32_t split_count(uint32_t L, uint32_t cpw) {
    const uint32_t tps = kWavesPerWg * cpw * kChunk;
    return (L + tps - 1) / tps;
}

// Cross-split combine.  Workgroup (sequence * kv_heads + head, block of 32
// consecutive output elements, all in one query-head row) holds one record slot per
// thread group: thread (q = tid & 7, rg = tid >> 3) reads elements 4q..4q+3 of records
// rg, rg + 32, rg + 64 (issued before the context length arrives, so one memory round
// trip covers a single sequence's 64 splits and the fused append's record) and of any
// further ones after it, folding them with its own running max.  The 32 record groups
// are then merged in a fixed butterfly (lanes 8, 16, 32 apart) and across the four
// waves in LDS, so the result is deterministic.
// Fused append (APPEND): the splits covered the L-1 cached keys and decode_kernel
// wrote the new token's record (m = score, l = 1, O = its dequantised V row) at
// slot nsplit, merged here as one more record.  The merge follows the reference
// combine (gfx906/kernels/qwen3_primitives.hip:2295-2385).
__device__ __forceinline__ void merge_state(float& m, float& l, float4& acc, float m2, float l2, float4 a2) {
    if (m2 == -INFINITY) return;
    if (m == -INFINITY) {
        m = m2; l = l2; acc = a2;
        return;
    }
    const float mn = fmaxf(m, m2);
    const float f1 = exp2_safe(m - mn), f2 = exp2_safe(m2 - mn);
    m = mn;
    l = l * f1 + l2 * f2;
    acc.x = acc.x * f1 + a2.x * f2;
    acc.y = acc.y * f1 + a2.y * f2;
    acc.z = acc.z * f1 + a2.z * f2;
    acc.w = acc.w * f1 + a2.w * f2;
}

// Gate values of elements i..i+3.  Called after the record loads are issued: a load
// in a branch is waited for at the branch's end, which would otherwise hold back the
// loads issued after it (here everything it waits for is needed next).
__device__ __forceinline__ void combine_gate(const SplitArgs& a, size_t i, float (&gv)[4]) {
    gv[0] = gv[1] = gv[2] = gv[3] = 0.0f;
    if (a.gate != nullptr) {
        const float4 g4 = *reinterpret_cast<const float4*>(a.gate + i);
        gv[0] = g4.x; gv[1] = g4.y; gv[2] = g4.z; gv[3] = g4.w;
    }
}

// Output of 4 merged elements e..e+3 (thread q of the 8 holding a 32-value block that
// starts at element blk0 of the launch's rows): out = acc / L, 0 when L == 0
// (qwen3_primitives.hip:2349); gated = out * sigmoid(gate); the Q8_1 block.  All 8
// threads of a block call it (the block's reductions); `live` = false computes but
// stores nothing.
__device__ __forceinline__ void combine_emit(const SplitArgs& a, size_t out_row0, uint32_t e, uint32_t q, size_t blk0,
                                             float l, float4 acc, const float (&gv)[4], bool live) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const float vals[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
    float gated[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.out && live) *reinterpret_cast<float4*>(a.out + out_row0 + e) = make_float4(vals[0], vals[1], vals[2], vals[3]);
    if (a.gate) {
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) gated[k] = vals[k] * (1.0f / (1.0f + expf(-gv[k])));
        if (a.gated_out && live)
            *reinterpret_cast<float4*>(a.gated_out + out_row0 + e) = make_float4(gated[0], gated[1], gated[2], gated[3]);
    }
    if (a.gate && a.gated_q8_1) {
        // Q8_1 block of these 32 gated values (qwen3_primitives.hip:2354-2384):
        // d = amax/127, q = clamp(roundf(x/d), -127, 127), s = sum(q)*d.
        float amax = fmaxf(fmaxf(fabsf(gated[0]), fabsf(gated[1])), fmaxf(fabsf(gated[2]), fabsf(gated[3])));
        amax = group_reduce<8>(amax, MaxOp{});
        const float d = amax / 127.0f;
        const float qinv = d != 0.0f ? 1.0f / d : 0.0f;
        int qs[4];
        int sum = 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) {
            qs[k] = max(-127, min(127, static_cast<int>(roundf(gated[k] * qinv))));
            sum += qs[k];
        }
        sum = group_reduce<8>(sum, AddOp{});
        if (!live) return;
        const size_t blk = (out_row0 + blk0) / 32;
        uint8_t* bp = a.gated_q8_1 + blk * 36;
        *reinterpret_cast<uint32_t*>(bp + 4 + 4 * q) =
            (static_cast<uint32_t>(qs[0]) & 0xffu) | ((static_cast<uint32_t>(qs[1]) & 0xffu) << 8) |
            ((static_cast<uint32_t>(qs[2]) & 0xffu) << 16) | ((static_cast<uint32_t>(qs[3]) & 0xffu) << 24);
        if (q == 0) {
            *reinterpret_cast<uint16_t*>(bp) = f32_to_f16_bits(d);
            *reinterpret_cast<uint16_t*>(bp + 2) = f32_to_f16_bits(static_cast<float>(sum) * d);
        }
    }
}


template <uint32_t D, bool APPEND>
__global__ void __launch_bounds__(256) combine_kernel(SplitArgs a) {
    const uint32_t bh = blockIdx.x;
    const uint32_t b = bh / a.g.kv_heads;
    const uint32_t h = bh % a.g.kv_heads;
    const uint32_t G = a.group;
    const uint32_t GD = G * D;
    const uint32_t tid = threadIdx.x;
    const uint32_t q = tid & 7, rg = tid >> 3;
    const uint32_t e = blockIdx.y * 32 + 4 * q;  // < GD: the grid covers GD / 32 blocks
    const uint32_t hn = (blockIdx.y * 32) / D;
    // output row of column hn (packed tokens: token pack*b + hn / Gt, head h*Gt + hn % Gt),
    // indexed below with the column's offset e - hn * D folded back in
    const uint32_t Gt = G / a.pack, tp = hn / Gt;
    const size_t out_row0 = ((static_cast<size_t>(b) * a.pack + tp) * a.q_heads + static_cast<size_t>(h) * Gt +
                             (hn - tp * Gt)) * D - static_cast<size_t>(hn) * D;
    const uint32_t rec = record_floats(G, D);
    const uint32_t slots = a.max_splits + 1;
    const float* part = a.part + (static_cast<size_t>(bh) * slots) * rec;

    constexpr uint32_t kSpec = 3;
    float ms[kSpec], ls[kSpec];
    float4 vv[kSpec];
#pragma unroll
    for (uint32_t j = 0; j < kSpec; ++j) {
        const uint32_t sp = rg + 32 * j;
        ms[j] = -INFINITY;
        ls[j] = 0.0f;
        vv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (sp < slots) {
            const float* r = part + static_cast<size_t>(sp) * rec;
            ms[j] = r[GD + hn];
            ls[j] = r[GD + G + hn];
            vv[j] = *reinterpret_cast<const float4*>(r + e);
        }
    }
    float gv[4];
    combine_gate(a, out_row0 + e, gv);
    const uint32_t cpw = launch_cpw(a);
    if (a.count_ptr != nullptr && b >= *a.count_ptr) return;
    const uint32_t L = split_length(a, b);
    const uint32_t nrec = split_count(L, cpw) + (APPEND && L > 0 ? 1u : 0u);

    float m = -INFINITY, l = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (uint32_t j = 0; j < kSpec; ++j)
        if (rg + 32 * j < nrec) merge_state(m, l, acc, ms[j], ls[j], vv[j]);
    for (uint32_t sp = rg + 32 * kSpec; sp < nrec; sp += 32) {
        const float* r = part + static_cast<size_t>(sp) * rec;
        merge_state(m, l, acc, r[GD + hn], r[GD + G + hn], *reinterpret_cast<const float4*>(r + e));
    }
    // Butterfly over the 8 record groups of this wave (lanes 8, 16, 32 apart).
#pragma unroll
    for (uint32_t off = 8; off < 64; off <<= 1) {
        const float m2 = __shfl_xor(m, off), l2 = __shfl_xor(l, off);
        float4 a2;
        a2.x = __shfl_xor(acc.x, off);
        a2.y = __shfl_xor(acc.y, off);
        a2.z = __shfl_xor(acc.z, off);
        a2.w = __shfl_xor(acc.w, off);
        merge_state(m, l, acc, m2, l2, a2);
    }
    __shared__ float4 s_acc[4][8];
    __shared__ float s_m[4][8], s_l[4][8];
    const uint32_t wave = tid >> 6;
    if ((tid & 63) < 8) {
        s_acc[wave][q] = acc;
        s_m[wave][q] = m;
        s_l[wave][q] = l;
    }
    __syncthreads();
    if (tid >= 8) return;
#pragma unroll
    for (uint32_t w = 1; w < 4; ++w) merge_state(m, l, acc, s_m[w][q], s_l[w][q], s_acc[w][q]);
    combine_emit(a, out_row0, e, q, blockIdx.y * 32, l, acc, gv, true);
}


// Cross-split combine for launches with few records per row set or many row sets:
// one thread per 4 consecutive outputs of one (row set, kv head) folds all of that row
// set's records itself, kNarrowRecords loads in flight at a time, so the grid is one
// thread per 4 outputs instead of a 256-thread workgroup per 32; 8 consecutive threads
// hold one 32-value block (Q8_1 epilogue).
constexpr uint32_t kNarrowRecords = 8;
template <uint32_t D, bool APPEND>
__global__ void __launch_bounds__(256) combine_narrow_kernel(SplitArgs a) {
    const uint32_t G = a.group;
    const uint32_t GD = G * D;
    const uint64_t idx = static_cast<uint64_t>(blockIdx.x) * 256 + threadIdx.x;
    const uint64_t per = GD / 4;
    const uint32_t bh = static_cast<uint32_t>(idx / per);
    const bool live = bh < a.batch * a.g.kv_heads;
    const uint32_t bhc = live ? bh : 0;
    const uint32_t b = bhc / a.g.kv_heads;
    const uint32_t h = bhc % a.g.kv_heads;
    const uint32_t e = static_cast<uint32_t>(idx % per) * 4;
    const uint32_t q = (e / 4) & 7;
    const uint32_t hn = e / D;
    const uint32_t Gt = G / a.pack, tp = hn / Gt;
    const size_t out_row0 = ((static_cast<size_t>(b) * a.pack + tp) * a.q_heads + static_cast<size_t>(h) * Gt +
                             (hn - tp * Gt)) * D - static_cast<size_t>(hn) * D;
    const uint32_t rec = record_floats(G, D);
    const float* part = a.part + (static_cast<size_t>(bhc) * (a.max_splits + 1)) * rec;
    // The first batch of record slots is read before the context length arrives (slots
    // past the row set's count hold stale bytes and are dropped below), then the gate.
    const uint32_t slots = a.max_splits + 1;
    float ms[kNarrowRecords], ls[kNarrowRecords];
    float4 vv[kNarrowRecords];
#pragma unroll
    for (uint32_t j = 0; j < kNarrowRecords; ++j) {
        if (j < slots) {
            const float* r = part + static_cast<size_t>(j) * rec;
            ms[j] = r[GD + hn];
            ls[j] = r[GD + G + hn];
            vv[j] = *reinterpret_cast<const float4*>(r + e);
        }
    }
    float gv[4];
    combine_gate(a, out_row0 + e, gv);
    // steps per wave (every thread of the workgroup takes part) with the loads in flight
    const uint32_t cpw = launch_cpw(a);
    // a whole 32-value block shares b (GD is a multiple of 32), so the 8 threads of a
    // block take the same exit
    if (a.count_ptr != nullptr && b >= *a.count_ptr) return;
    const uint32_t L = split_length(a, b);
    const uint32_t nrec = split_count(L, cpw) + (APPEND && L > 0 ? 1u : 0u);
    float m = -INFINITY, l = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (uint32_t j = 0; j < kNarrowRecords; ++j)
        if (j < nrec) merge_state(m, l, acc, ms[j], ls[j], vv[j]);
    for (uint32_t sp0 = kNarrowRecords; sp0 < nrec; sp0 += kNarrowRecords) {  // further batches
#pragma unroll
        for (uint32_t j = 0; j < kNarrowRecords; ++j) {
            ms[j] = -INFINITY;
            if (sp0 + j < nrec) {
                const float* r = part + static_cast<size_t>(sp0 + j) * rec;
                ms[j] = r[GD + hn];
                ls[j] = r[GD + G + hn];
                vv[j] = *reinterpret_cast<const float4*>(r + e);
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < kNarrowRecords; ++j)
            if (sp0 + j < nrec) merge_state(m, l, acc, ms[j], ls[j], vv[j]);
    }
    combine_emit(a, out_row0, e, q, e - 4 * q, l, acc, gv, live);
}

}  // namespace
}  // namespace miikv
