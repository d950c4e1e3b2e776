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
    uint32_t group;  // query heads per kv head (<= 16)
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
    uint32_t q_f32;         // q dtype (scoring the appended token)
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
// fit in one round of `slots` resident workgroups.  Called by all threads of a
// 256-thread block (barriers inside).
__device__ uint32_t launch_cpw(const SplitArgs& a) {
    if (a.batch == 1 || a.slots == 0) return a.cpw;
    __shared__ unsigned long long s_sum[256];
    const uint32_t tid = threadIdx.x;
    const uint32_t count = a.count_ptr ? min(a.batch, *a.count_ptr) : a.batch;
    unsigned long long sum = 0;
    for (uint32_t bb = tid; bb < count; bb += 256) sum += split_length(a, bb);
    s_sum[tid] = sum;
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
    return static_cast<uint32_t>(cpw < a.cpw ? a.cpw : (cpw > 64 ? 64 : cpw));
}

// Split count of sequence b at `cpw` steps per wave (0 when L == 0).
__device__ __forceinline__ uint32_t split_count(uint32_t L, uint32_t cpw) {
    const uint32_t tps = kWavesPerWg * cpw * kChunk;
    return (L + tps - 1) / tps;
}

// Cross-split combine.  Workgroup (sequence * kv_heads + head, element block of 64)
// reads the partial records of every split of that (sequence, kv head): thread
// (e4 = tid & 15, sg = tid >> 4) folds records sg, sg+16, ... for 4 consecutive
// elements with its own running max, so its loads are independent; the 16 split
// groups are merged in a fixed order through LDS (deterministic result).
// Fused append (APPEND): the splits covered the L-1 cached keys and decode_kernel
// wrote the new token's record (m = score, l = 1, O = its dequantised V row) at
// slot nsplit, merged here as one more record.
template <uint32_t D, bool APPEND>
__global__ void __launch_bounds__(256) combine_kernel(SplitArgs a) {
    const uint32_t bh = blockIdx.x;
    const uint32_t b = bh / a.g.kv_heads;
    const uint32_t h = bh % a.g.kv_heads;
    const uint32_t G = a.group;
    const uint32_t GD = G * D;
    const uint32_t e0 = blockIdx.y * 64;
    if (e0 >= GD) return;
    const uint32_t tid = threadIdx.x;
    const uint32_t e4 = tid & 15;
    const uint32_t sg = tid >> 4;
    const uint32_t e = e0 + e4 * 4;
    const bool active = e < GD;
    const uint32_t hn = active ? e / D : 0;
    const size_t out_row0 = (static_cast<size_t>(b) * a.q_heads + static_cast<size_t>(h) * G) * D;

    const uint32_t rec = record_floats(G, D);
    const uint32_t slots = a.max_splits + 1;
    const float* part = a.part + (static_cast<size_t>(bh) * slots) * rec;

    // The first kSpec records of this thread are fetched before the context length
    // (and with it the record count) arrives; records past the count are ignored.
    // 16 * kSpec = 80 covers a single sequence's 64 splits plus the fused append's
    // record, so none of them waits for the length (a 65th record fetched after it
    // added one dependent memory round trip to the combine).
#ifndef MIIKV_COMBINE_SPEC
#define MIIKV_COMBINE_SPEC 5
#endif
    constexpr uint32_t kSpec = MIIKV_COMBINE_SPEC;
    // The gate of this thread's outputs (split group 0 writes them) goes out with the
    // records, so the epilogue does not wait for it.
    float gv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.gate != nullptr && sg == 0 && active) {
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) gv[k] = a.gate[out_row0 + e + k];
    }
    float ms[kSpec], ls[kSpec];
    float4 vv[kSpec];
#pragma unroll
    for (uint32_t j = 0; j < kSpec; ++j) {
        const uint32_t sp = sg + 16 * j;
        ms[j] = -INFINITY;
        ls[j] = 0.0f;
        vv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (sp < slots) {
            const float* r = part + static_cast<size_t>(sp) * rec;
            ms[j] = r[GD + hn];
            ls[j] = r[GD + G + hn];
            if (active) vv[j] = *reinterpret_cast<const float4*>(r + e);
        }
    }
    const uint32_t cpw = launch_cpw(a);
    if (a.count_ptr != nullptr && b >= *a.count_ptr) return;
    const uint32_t L = split_length(a, b);
    const uint32_t nrec = split_count(L, cpw) + (APPEND && L > 0 ? 1u : 0u);

    float mloc = -INFINITY;
    float lsum = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto merge = [&](float m_s, float l_s, float4 v) {
        if (m_s == -INFINITY) return;  // a split with no key (possible with the fused append)
        const float mn = fmaxf(mloc, m_s);
        const float fo = exp2_safe(mloc - mn);  // 0 on the first split
        const float fs = exp2_safe(m_s - mn);
        mloc = mn;
        lsum = lsum * fo + l_s * fs;
        acc.x = acc.x * fo + v.x * fs;
        acc.y = acc.y * fo + v.y * fs;
        acc.z = acc.z * fo + v.z * fs;
        acc.w = acc.w * fo + v.w * fs;
    };
#pragma unroll
    for (uint32_t j = 0; j < kSpec; ++j)
        if (sg + 16 * j < nrec) merge(ms[j], ls[j], vv[j]);
    for (uint32_t sp = sg + 16 * kSpec; sp < nrec; sp += 16) {
        const float* r = part + static_cast<size_t>(sp) * rec;
        merge(r[GD + hn], r[GD + G + hn],
              active ? *reinterpret_cast<const float4*>(r + e) : make_float4(0.f, 0.f, 0.f, 0.f));
    }
    __shared__ float4 s_acc[16][16];
    __shared__ float s_gm[16][16];
    __shared__ float s_gl[16][16];
    s_acc[sg][e4] = acc;
    s_gm[sg][e4] = mloc;
    s_gl[sg][e4] = lsum;
    __syncthreads();
    if (sg != 0 || !active) return;
    float M = -INFINITY;
#pragma unroll
    for (uint32_t g = 0; g < 16; ++g) M = fmaxf(M, s_gm[g][e4]);
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float Ls = 0.0f;
#pragma unroll
    for (uint32_t g = 0; g < 16; ++g) {
        const float mg = s_gm[g][e4];
        if (mg == -INFINITY) continue;  // split group without splits
        const float f = exp2_safe(mg - M);
        const float4 v = s_acc[g][e4];
        o.x += f * v.x;
        o.y += f * v.y;
        o.z += f * v.z;
        o.w += f * v.w;
        Ls += f * s_gl[g][e4];
    }
    // out = acc / L, 0 when L == 0 (qwen3_primitives.hip:2349); gated = out * sigmoid(gate).
    const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
    const float vals[4] = {o.x * inv, o.y * inv, o.z * inv, o.w * inv};
    float gated[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        const size_t oi = out_row0 + e + k;
        if (a.out) a.out[oi] = vals[k];
        if (a.gate) {
            gated[k] = vals[k] * (1.0f / (1.0f + expf(-gv[k])));
            if (a.gated_out) a.gated_out[oi] = gated[k];
        }
    }
    if (a.gate && a.gated_q8_1) {
        // Q8_1 block of 32 gated values = 8 consecutive lanes (qwen3_primitives.hip:
        // 2354-2384): d = amax/127, q = clamp(roundf(x/d), -127, 127), s = sum(q)*d.
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
        const size_t blk = (out_row0 + e) / 32;
        uint8_t* bp = a.gated_q8_1 + blk * 36;
        *reinterpret_cast<uint32_t*>(bp + 4 + 4 * (e4 & 7)) =
            (static_cast<uint32_t>(qs[0]) & 0xffu) | ((static_cast<uint32_t>(qs[1]) & 0xffu) << 8) |
            ((static_cast<uint32_t>(qs[2]) & 0xffu) << 16) | ((static_cast<uint32_t>(qs[3]) & 0xffu) << 24);
        if ((e4 & 7) == 0) {
            *reinterpret_cast<uint16_t*>(bp) = f32_to_f16_bits(d);
            *reinterpret_cast<uint16_t*>(bp + 2) = f32_to_f16_bits(static_cast<float>(sum) * d);
        }
    }
}

}  // namespace
}  // namespace miikv
