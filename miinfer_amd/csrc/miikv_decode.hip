// Split-K GQA decode attention over the tiled q8_0 cache (gfx950, wave64, MFMA).
//
// Work decomposition.  A workgroup of 4 waves owns one (sequence, kv head,
// split); a split is 4 * cpw steps of 32 tokens and each wave streams cpw
// consecutive steps.  All G = q_heads / kv_heads query heads of the kv head are
// served by the same wave, so every K/V byte is read from HBM exactly once.
//
// Per 32-token step a wave computes, for its 2 tiles of 16 tokens:
//   S^T[token][head] = K_tile (16 x D, int8 -> fp16) * Q^T (D x 16 heads)
// with v_mfma_f32_16x16x32_f16, one MFMA per 32-value q8_0 block so the block
// scale is applied to the fp32 result (exact in the codes).  The output
// fragment (lane (g,n) holds tokens 4g..4g+3 of head n) is exactly the B
// operand layout of v_mfma_f32_16x16x16_f16, so after the online-softmax
// update the probabilities feed
//   O^T[dim][head] += V^T (16 dims x 16 tokens, int8 -> fp16) * P^T
// without any cross-lane movement; the V block scale is folded into P^T per
// block.  Softmax runs in the log2 domain (scores pre-multiplied by
// scale * log2(e)) with exp2.
//
// Cross-wave combine goes through LDS; each workgroup writes one partial record
// (m, l, unnormalised O) per split into the caller's workspace, and a second,
// wide kernel merges the splits.  Merging inside this launch instead (records
// written with device-scope stores, an arrival counter, the last arrivals
// merging) measured no faster: the merge then costs the counter's and the
// records' round trips on top of the last split, about what the second launch
// costs.  The merge follows the reference combine
// (gfx906/kernels/qwen3_primitives.hip:2295-2385): g = max m_s,
// L = sum l_s e^{m_s-g}, out = sum acc_s e^{m_s-g} / L, 0 when L == 0,
// gated = out * sigmoid(gate).  With the fused append, the last workgroups of
// the grid quantise, store and score the new token and write it as one more
// record (append_record).
#include "miikv_common.hpp"
#include "miikv_split.hpp"

#include <cmath>
#include <cstdlib>
#include <mutex>
#include <type_traits>

namespace miikv {

int validate_view(const miikv_view* v);
uint64_t view_seq_capacity(const miikv_view* v);

namespace {

// Pipeline depth (32-token steps held in registers) and the occupancy it is tuned for.
// D = 128: a single sequence's grid holds two waves per SIMD (kTargetWaves), so the
// second step buffer costs no occupancy there (config 2 at 32k: 21.8 -> 21.4 us).
#ifndef MIIKV_RING_D128
#define MIIKV_RING_D128 2
#endif
#ifndef MIIKV_WPE_D128
#define MIIKV_WPE_D128 2
#endif
#ifndef MIIKV_RING_F16_D128
#define MIIKV_RING_F16_D128 2
#endif
#ifndef MIIKV_RING_D256
#define MIIKV_RING_D256 1
#endif
#ifndef MIIKV_RING_D256_F32
#define MIIKV_RING_D256_F32 1
#endif
#ifndef MIIKV_WPE_D256_F32
#define MIIKV_WPE_D256_F32 1
#endif
#ifndef MIIKV_VBIAS_D256_F32
#define MIIKV_VBIAS_D256_F32 1
#endif
#ifndef MIIKV_WPE_D256
#define MIIKV_WPE_D256 2
#endif
#ifndef MIIKV_VBIAS_D256
#define MIIKV_VBIAS_D256 0
#endif
#ifndef MIIKV_VBIAS_D128
#define MIIKV_VBIAS_D128 1
#endif
#ifndef MIIKV_NT_SCALES_D128
#define MIIKV_NT_SCALES_D128 1
#endif
#ifndef MIIKV_NT_SCALES_D256
#define MIIKV_NT_SCALES_D256 0
#endif
// An fp32 query carries a second (low-half) set of query fragments and a second
// MFMA per block; those variants keep a deeper ring at lower occupancy.
template <uint32_t D, bool QF32>
struct DecodeTuning {
    static constexpr uint32_t ring = D == 128 ? MIIKV_RING_D128 : (QF32 ? MIIKV_RING_D256_F32 : MIIKV_RING_D256);
    static constexpr uint32_t waves_per_eu = D == 128 ? (QF32 ? 2 : MIIKV_WPE_D128) : (QF32 ? MIIKV_WPE_D256_F32 : MIIKV_WPE_D256);
    static constexpr bool vbias = D == 128 ? MIIKV_VBIAS_D128 != 0 : (QF32 ? MIIKV_VBIAS_D256_F32 != 0 : MIIKV_VBIAS_D256 != 0);
    // Nontemporal scale loads: config 2 (D = 128) at 32k 20.5 -> 20.2 us; config 3
    // (D = 256) 157 -> 160 us, so cached there.
    static constexpr bool nt_scales = D == 128 ? MIIKV_NT_SCALES_D128 != 0 : MIIKV_NT_SCALES_D256 != 0;
};
constexpr uint32_t kTargetWaves = 256 * 8;  // 256 CUs x 8 resident waves
#ifndef MIIKV_INTERLEAVE_CPW
#define MIIKV_INTERLEAVE_CPW 4
#endif
constexpr uint32_t kInterleaveCpw = MIIKV_INTERLEAVE_CPW;  // steps per wave at which waves interleave
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kCodeBias = 1152.0f;  // codes enter the MFMA as fp16(code + 1152)
constexpr float kRescaleSlack = 6.0f;  // log2 units: p <= 64, and 64 * (65504/127) < 65504


// Streaming loads of cache codes: each byte is read once per launch, so they are
// issued nontemporal (measured ~5% faster than cached loads at 32k context).
// CACHED: row sets of one sequence (a suffix run as decodes) read the same keys, and
// the workgroups of one XCD run the row sets of one key range together, so the codes
// are loaded through the L2 for the other row sets to find.
template <bool CACHED = false>
__device__ __forceinline__ uint4 load16(const int8_t* p) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v t = CACHED ? *reinterpret_cast<const u4v*>(p) : __builtin_nontemporal_load(reinterpret_cast<const u4v*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
template <bool CACHED = false>
__device__ __forceinline__ uint2 load8(const int8_t* p) {
    typedef unsigned int u2v __attribute__((ext_vector_type(2)));
    const u2v t = CACHED ? *reinterpret_cast<const u2v*>(p) : __builtin_nontemporal_load(reinterpret_cast<const u2v*>(p));
    return make_uint2(t.x, t.y);
}

// One lane's NB/2 block scales of a step; NT: nontemporal, like the codes.
template <typename T, bool NT>
__device__ __forceinline__ T load_scales(const uint16_t* p) {
    if constexpr (!NT) {
        return *reinterpret_cast<const T*>(p);
    } else if constexpr (sizeof(T) == 4) {
        return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
    } else {
        typedef unsigned int u2v __attribute__((ext_vector_type(2)));
        const u2v t = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(p));
        return T{t.x, t.y};
    }
}

__device__ __forceinline__ float wave_max_xor_16_32(float x) {
    return rows_reduce(x, MaxOp{});
}

// Raw v_exp_f32: no denormal range fix-up (results below 2^-126 flush to 0, which
// only drops probabilities that are already negligible); exp2(-inf) == 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }


// Packed work items of a batch: sequence b owns ceil(L_b / split tokens) * kv_heads
// items (none past *count_ptr).  Every workgroup scans the per-sequence counts
// (256 sequences per pass, Hillis-Steele in LDS) and finds the item at index
// `id`; false if the batch holds fewer items.  Called by every thread of the
// workgroup (barriers inside); the first 256 threads do the scan.
__device__ bool locate_item(const SplitArgs& a, uint32_t cpw, uint32_t id, uint32_t& b_out, uint32_t& h_out,
                            uint32_t& split_out) {
    __shared__ uint32_t s_scan[256];
    __shared__ uint32_t s_hit[3];
    const uint32_t tid = threadIdx.x;
    const uint32_t tps = kWavesPerWg * cpw * kChunk;
    const uint32_t H = a.g.kv_heads;
    const uint32_t count = a.count_ptr ? min(a.batch, *a.count_ptr) : a.batch;
    if (tid == 0) s_hit[0] = 0xffffffffu;
    uint32_t base = 0;
    const bool scans = tid < 256;
    for (uint32_t b0 = 0; b0 < count; b0 += 256) {
        const uint32_t bb = b0 + tid;
        const uint32_t nsplit = scans && bb < count ? (split_length(a, bb) + tps - 1) / tps : 0;
        const uint32_t n = nsplit * H;
        if (scans) s_scan[tid] = n;
        __syncthreads();
        for (uint32_t off = 1; off < 256; off <<= 1) {
            const uint32_t add = scans && tid >= off ? s_scan[tid - off] : 0;
            __syncthreads();
            if (scans) s_scan[tid] += add;
            __syncthreads();
        }
        const uint32_t incl = base + (scans ? s_scan[tid] : 0);
        const uint32_t excl = incl - n;
        if (scans && id >= excl && id < incl) {
            const uint32_t rem = id - excl;
            s_hit[0] = bb;
            s_hit[1] = rem / nsplit;
            s_hit[2] = rem % nsplit;
        }
        base += s_scan[255];
        __syncthreads();
    }
    __syncthreads();
    if (s_hit[0] == 0xffffffffu) return false;
    b_out = s_hit[0];
    h_out = s_hit[1];
    split_out = s_hit[2];
    return true;
}

// The reference's K prologue for one row held one value per thread (thread t < D owns
// dim t), in its own shape (qwen35_decoupled_k_norm_rope_kv_store_batch_quant_kernel,
// gfx906/kernels/qwen3_primitives.hip:7257-7281): sum of squares by the tree
// p[t] += p[t + stride], stride = D/2 .. 1; value * (1 / sqrt(ss / D + eps)) * weight;
// pairs (t, t + 32), t < 32, rotated by position * step^t.  Same additions in the same
// order as miikv_append_f32's prologue, so the stored codes are the same.  Here the
// levels that cross waves (strides >= 64) are formed by every wave from one LDS
// exchange, the levels within a wave with shuffles, and each rotation pair (32 lanes
// apart in wave 0) with one swap, so the whole prologue costs one barrier.  Called by
// all 256 threads.
template <uint32_t D>
__device__ void k_prologue(float& kx, float w, uint32_t tid, uint32_t position, float step, float eps) {
#pragma clang fp contract(off)
    static_assert(D == 128 || D == 256, "the tree's cross-wave levels are written for D = 128 and 256");
    __shared__ float s_p[256];
    const uint32_t lane = tid & 63;
    s_p[tid] = tid < D ? kx * kx : 0.0f;
    __syncthreads();
    float p;  // p[lane] after the levels of stride >= 64 (the same value in every wave)
    if constexpr (D == 256) {
        const float a0 = s_p[lane] + s_p[lane + 128], a1 = s_p[lane + 64] + s_p[lane + 192];
        p = a0 + a1;
    } else {
        p = s_p[lane] + s_p[lane + 64];
    }
#pragma unroll
    for (uint32_t stride = 32; stride > 0; stride >>= 1) p = p + __shfl_down(p, stride, 64);
    const float ss = __shfl(p, 0, 64);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
    kx = kx * r * w;
    if (tid < 64) {
        // position * step * step ... ((tid & 31) factors, in that order), unrolled with
        // selects rather than a loop whose trip count differs per lane
        float angle = static_cast<float>(position);
#pragma unroll
        for (uint32_t i = 0; i < 31; ++i) {
            const float next = angle * step;
            angle = i < (tid & 31) ? next : angle;
        }
        float sn, cs;
        rope_sincos(angle, &sn, &cs);
        const float other = __shfl_xor(kx, 32, 64);
        kx = tid < 32 ? kx * cs - other * sn : other * sn + kx * cs;
    }
    __syncthreads();  // s_p is reused by the next call
}

// Fused append for (sequence b, kv head h), by one 256-thread workgroup: quantise
// the new fp16 K/V rows with the append rule (thread t < D owns dim t; block absmax
// over 32 lanes), store them at position L-1, score the K row against the G query
// heads, and write the token's record (m = score, l = 1, O = dequantised V row for
// every head) at slot nsplit, after the splits, which cover the L-1 cached keys.
// The row and query loads go out before the context length arrives.
template <uint32_t D>
__device__ void append_record(const SplitArgs& a, uint32_t b, uint32_t h, uint32_t cpw) {
    constexpr uint32_t DJ = D / 64;
    __shared__ float s_k[D];
    __shared__ float s_v[D];
    __shared__ float s_score[16];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t G = a.group;
    // Threads past D (whole waves: D is a multiple of 64) load dim D-1 and discard it.
    const uint32_t t = min(tid, D - 1);
    const size_t row = (static_cast<size_t>(b) * a.g.kv_heads + h) * D + t;
    const bool rows32 = a.k_new32 != nullptr;
    float kx = rows32 ? a.k_new32[row] : f16_bits_to_f32(a.k_new[row]);
    const float vx = rows32 ? a.v_new32[row] : f16_bits_to_f32(a.v_new[row]);
    const float kw = a.k_norm_weight != nullptr ? a.k_norm_weight[t] : 0.0f;
    // Wave w scores heads w, w+4, ... with dims lane + 64j; an fp16 query is read as
    // the 32-bit word holding the value (one load form for both query types).
    uint32_t qw[4][DJ];
    const uint32_t* q32 = static_cast<const uint32_t*>(a.q);
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t g = min(wave + 4 * j, G - 1);
        const size_t qi = (static_cast<size_t>(b) * a.q_heads + static_cast<size_t>(h) * G + g) * D + lane;
#pragma unroll
        for (uint32_t jj = 0; jj < DJ; ++jj) qw[j][jj] = q32[a.q_f32 ? qi + 64 * jj : (qi + 64 * jj) / 2];
    }
    const uint32_t L = split_length(a, b);
    if (L == 0) return;  // no token (the combine writes zeros)
    if (a.k_norm_weight != nullptr) k_prologue<D>(kx, kw, tid, L - 1, a.rope_step, a.epsilon);
    const float ka = group_reduce<32>(fabsf(kx), MaxOp{});
    const float va = group_reduce<32>(fabsf(vx), MaxOp{});
    const float ksc = ka > 0.0f ? ka / 127.0f : 1.0f, vsc = va > 0.0f ? va / 127.0f : 1.0f;
    const int kq = max(-128, min(127, __float2int_rn(kx * (1.0f / ksc))));
    const int vq = max(-128, min(127, __float2int_rn(vx * (1.0f / vsc))));
    const uint16_t kbits = f32_to_f16_bits(ksc), vbits = f32_to_f16_bits(vsc);
    if (tid < D) {
        s_k[tid] = static_cast<float>(kq) * f16_bits_to_f32(kbits);
        s_v[tid] = static_cast<float>(vq) * f16_bits_to_f32(vbits);
        const uint32_t pos = L - 1;
        const size_t slab = slab_of(a.g, b, pos, h);
        const uint32_t tp = pos % a.g.page_tokens;
        const size_t slab_bytes = static_cast<size_t>(a.g.page_tokens) * D;
        a.g.k_codes[slab * slab_bytes + k_code_offset(tp, tid & ~7u, D) + (tid & 7u)] = static_cast<int8_t>(kq);
        a.g.v_codes[slab * slab_bytes + v_code_offset(tp, tid, D)] = static_cast<int8_t>(vq);
        if ((tid & 31) == 0) {
            const size_t sidx = (slab * a.g.page_tokens + tp) * (D / 32) + tid / 32;
            a.g.k_scales[sidx] = kbits;
            a.g.v_scales[sidx] = vbits;
        }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint32_t g = wave + 4 * j;
        if (g >= G) break;  // wave-uniform
        float dot = 0.0f;
#pragma unroll
        for (uint32_t jj = 0; jj < DJ; ++jj) {
            const uint32_t w = qw[j][jj];
            const float qx = a.q_f32 ? __uint_as_float(w) : f16_bits_to_f32(static_cast<uint16_t>((lane & 1) ? w >> 16 : w));
            dot += qx * s_k[lane + 64 * jj];
        }
        dot = group_reduce<64>(dot, AddOp{});
        if (lane == 0) s_score[g] = dot * a.scale_log2;
    }
    __syncthreads();
    const uint32_t rec = record_floats(G, D);
    float* r = a.part + ((static_cast<size_t>(b) * a.g.kv_heads + h) * (a.max_splits + 1) + split_count(L, cpw)) * rec;
    for (uint32_t i4 = tid; i4 < G * D / 4; i4 += 256) {
        const uint32_t d = (4 * i4) % D;
        *reinterpret_cast<float4*>(r + 4 * i4) = make_float4(s_v[d], s_v[d + 1], s_v[d + 2], s_v[d + 3]);
    }
    if (tid < G) {
        r[G * D + tid] = s_score[tid];
        r[G * D + G + tid] = 1.0f;
    }
    __syncthreads();  // the caller reuses the LDS
}

// KF16 / VF16: the K / V plane holds fp16 rows (quant modes FP16_*, the reference's
// control path, qwen3_wave64_splitk_stage1_f16_kernel at qwen3_primitives.hip:2198-2293):
// the fragments are loaded as fp16 and enter the MFMAs unscaled.  fp16 fragments take
// twice the registers: D = 128 runs a two-step ring at two waves per SIMD (config 2,
// FP16_FP16: 27.4 -> 26.7 us against one step at three), D = 256 (and a second query
// fragment set) one step.
// Waves per SIMD of a decode_kernel instance: the tuned value, except q8 keys with fp16
// values at D = 256, which need a wave's full register file (two waves spilled 122).
// Lane n of a row of 16 takes the value of lane n + K (DPP row_shl; 0 past the row).
template <uint32_t K>
__device__ __forceinline__ float dpp_row_shl(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x100 + K, 0xF, 0xF,
                                                                 false));
}
template <uint32_t D, bool QF32, bool KF16, bool VF16>
constexpr uint32_t decode_waves_per_eu() {
    return (D == 256 && VF16 && !KF16) ? 1u : DecodeTuning<D, QF32>::waves_per_eu;
}
// An fp32 query is split into fp16 hi + lo parts.  QPAIR (G <= 8): the lo parts ride in
// the QK MFMA's unused columns 8..8+G-1 (B operand column 8 + g = lo of head g), so one
// MFMA per block carries both and the two column sums meet with one 8-lane row shift
// per score (a constant DPP shift); the fp16-query register budget and occupancy then
// hold.  Otherwise (G > 8) the lo parts are a second fragment set and a second MFMA per
// block.
template <uint32_t D, bool QF32, bool APPEND, bool KF16 = false, bool VF16 = false, bool QPAIR = false,
          bool CACHED = false>
__global__ void __launch_bounds__(64 * kWavesPerWg)
__attribute__((amdgpu_waves_per_eu(decode_waves_per_eu<D, QF32 && !QPAIR, KF16, VF16>())))
decode_kernel(SplitArgs a) {
    constexpr uint32_t NB = D / 32;   // q8_0 blocks per row
    constexpr uint32_t NC = D / 64;   // 16-byte K loads per tile row group
    constexpr uint32_t NM = D / 16;   // V M-tiles (16 dims each)
    using ScaleVec = typename std::conditional<NB == 4, uint32_t, uint2>::type;  // NB/2 fp16 scales
    // V codes enter the PV MFMA biased (one v_perm per two codes) and the bias is removed
    // with column sums, or exactly (perm + subtract): the fold costs NB accumulators.
    constexpr bool kLo = QF32 && !QPAIR;  // separate lo fragments and MFMAs
    static_assert(!QPAIR || QF32, "QPAIR splits an fp32 query");
    constexpr bool kVBias = DecodeTuning<D, kLo>::vbias && !VF16;
    static_assert(!APPEND || (!KF16 && !VF16), "the fused append stores q8 rows");
    extern __shared__ float smem[];

    // Work item of this workgroup: one (sequence b, kv head h, split) of 4 waves x
    // cpw steps.  One sequence: workgroup x = h * max_splits + split.  A batch: the
    // items that hold keys are packed to the front of the grid (sequence-major,
    // then head, then split), so whatever the lengths, the busy workgroups are the
    // first ones dispatched and spread evenly over the XCDs and CUs; the grid's
    // tail (bounded by max_context) exits at once.
    const uint32_t cpw = launch_cpw(a);
    // Fused append: the last batch * kv_heads workgroups of the grid each handle the
    // new token of one (sequence, kv head).  Dispatched last, they take CU slots left
    // free by a small grid or freed by the first split workgroups to finish, so they
    // stay off the critical path.
    if constexpr (APPEND) {
        const uint32_t first = gridDim.x - a.batch * a.g.kv_heads;
        if (blockIdx.x >= first) {
            const uint32_t x = blockIdx.x - first;
            const uint32_t ab = x / a.g.kv_heads;
            if (a.count_ptr == nullptr || ab < *a.count_ptr) append_record<D>(a, ab, x % a.g.kv_heads, cpw);
            return;
        }
    }
    uint32_t split, h, b;
    if (a.rowset_order) {
        // Row sets of one sequence: items (kv head, split, row set), row sets fastest,
        // each XCD (workgroup i runs on XCD i % 8) a contiguous range of them, so the
        // workgroups an XCD runs together read the same keys (through its L2).  The
        // grid is padded to a multiple of 8; items past a row set's splits exit.
        const uint32_t total = a.max_splits * a.g.kv_heads * a.batch;
        const uint32_t k = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
        if (k >= total) return;
        b = k % a.batch;
        split = (k / a.batch) % a.max_splits;
        h = k / a.batch / a.max_splits;
        if (a.count_ptr != nullptr && b >= *a.count_ptr) return;
    } else if (a.batch == 1) {
        b = 0;
        h = blockIdx.x / a.max_splits;
        split = blockIdx.x % a.max_splits;
    } else if (!locate_item(a, cpw, blockIdx.x, b, h, split)) {
        return;
    }
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63;
    const uint32_t g4 = lane >> 4;
    const uint32_t n = lane & 15;
    const uint32_t G = a.group;
    const Geo& geo = a.g;

    // Steps this wave may own, from the host bound alone: the first loads are issued
    // before the context length arrives from memory.
    // A split is 4*cpw consecutive steps.  At cpw == kInterleaveCpw wave w takes
    // steps w, w+4, ... of it (the four waves of a workgroup then read one contiguous
    // region at a time); otherwise each wave streams the w-th run of cpw steps.  A
    // measured choice, not a model: config 2 shape, interleaved against runs, cpw 2
    // (16k) +0.3 us, cpw 4 (32k) -0.4 us, cpw 8 (64k) +0.15 us.  The wave's local
    // step i (0 <= i < n_steps) is split step first + i * stride.
    const uint32_t nsteps_max = (a.max_context + kChunk - 1) / kChunk;
    const bool interleave = cpw == kInterleaveCpw;
    const uint32_t stride = interleave ? kWavesPerWg : 1u;
    const uint32_t first = interleave ? split * kWavesPerWg * cpw + wave : (split * kWavesPerWg + wave) * cpw;
    const uint32_t last_excl = min(interleave ? (split + 1) * kWavesPerWg * cpw : first + cpw, nsteps_max);
    const uint32_t n_max = first < last_excl ? (last_excl - first + stride - 1) / stride : 0;
    const size_t slab_bytes = static_cast<size_t>(geo.page_tokens) * D;

    // Registers of one 32-token step: two K tiles, one V group, their scales.
    struct Step {
        uint4 k[2][NC][KF16 ? 2 : 1];                            // fp16: two words per fragment
        typename std::conditional<VF16, uint4, uint2>::type v[NM];  // fp16: 8 values per lane
        ScaleVec ks, vs;
    };

    // Load cursor: the page (slab) is looked up once per page, not per step.  Page
    // indices are clamped into the pool, so a speculative load past the sequence end
    // reads a valid (unused) page rather than whatever an unset table entry holds.
    uint32_t ld_tok = first * kChunk;
    uint32_t ld_tp = ld_tok % geo.page_tokens;
    size_t ld_slab = 0;
    if (n_max > 0) ld_slab = slab_of_clamped(geo, b, ld_tok, h);
    auto load_step = [&](Step& st) {
        if (ld_tp >= geo.page_tokens) {
            ld_tp = ld_tok % geo.page_tokens;
            ld_slab = slab_of_clamped(geo, b, ld_tok, h);
        }
        constexpr uint32_t KE = KF16 ? 2 : 1, VE = VF16 ? 2 : 1;  // bytes per element
        const int8_t* kb = geo.k_codes + (ld_slab * slab_bytes + static_cast<size_t>(ld_tp) * D) * KE;
        const int8_t* vb = geo.v_codes + (ld_slab * slab_bytes + static_cast<size_t>(ld_tp) * D) * VE;
        const size_t sc0 = (ld_slab * geo.page_tokens + ld_tp) * NB;
        // Scales first, each ahead of its codes: loads complete in issue order, so the
        // score MFMAs wait only for the K scales and codes while V is still in flight.
        if constexpr (!KF16)
            st.ks = load_scales<ScaleVec, DecodeTuning<D, kLo>::nt_scales && !CACHED>(geo.k_scales + sc0 + lane * (NB / 2));
#pragma unroll
        for (uint32_t J = 0; J < 2; ++J)
#pragma unroll
            for (uint32_t cc = 0; cc < NC; ++cc)
#pragma unroll
                for (uint32_t e = 0; e < KE; ++e)
                    st.k[J][cc][e] = load16<CACHED>(kb + KE * (J * 16 * D + cc * 1024 + g4 * 256 + n * 16) + 16 * e);
        if constexpr (!VF16)
            st.vs = load_scales<ScaleVec, DecodeTuning<D, kLo>::nt_scales && !CACHED>(geo.v_scales + sc0 + lane * (NB / 2));
#pragma unroll
        for (uint32_t mt = 0; mt < NM; ++mt) {
            if constexpr (VF16) st.v[mt] = load16<CACHED>(vb + 2 * ((16 * mt + n) * 32 + g4 * 8));
            else st.v[mt] = load8<CACHED>(vb + (16 * mt + n) * 32 + g4 * 8);
        }
        ld_tok += stride * kChunk;
        ld_tp += stride * kChunk;
    };

    // Ring of kRing step buffers; the first kRing-1 are loaded before L is known.
    constexpr uint32_t kRing = (KF16 || VF16) ? (D == 128 && !kLo ? MIIKV_RING_F16_D128 : 1u) : DecodeTuning<D, kLo>::ring;
    Step S[kRing];
#pragma unroll
    for (uint32_t r = 0; r + 1 < kRing; ++r)
        if (r < n_max) load_step(S[r]);

    // fp16 query bits, issued before the context length so that the two loads
    // overlap (lanes past the group read the group's last head and discard it).
    uint4 qraw[QF32 ? 1 : NB];
    float4 q32raw[QF32 ? NB : 1][2];
    {
        const uint32_t qh = QPAIR && n >= 8 ? min(n - 8, G - 1) : min(n, G - 1);
        // packed tokens (a short suffix): column qh is token pack*b + qh / Gt, head qh % Gt
        const uint32_t Gt = a.pack == 1 ? G : G / a.pack;
        const uint32_t tp = a.pack == 1 ? 0u : qh / Gt;
        const size_t qrow = ((static_cast<size_t>(b) * a.pack + tp) * a.q_heads + static_cast<size_t>(h) * Gt +
                             (qh - tp * Gt)) * D;
#pragma unroll
        for (uint32_t blk = 0; blk < NB; ++blk) {
            if constexpr (QF32) {
                const float* qp = static_cast<const float*>(a.q) + qrow + blk * 32 + g4 * 8;
                q32raw[blk][0] = *reinterpret_cast<const float4*>(qp);
                q32raw[blk][1] = *reinterpret_cast<const float4*>(qp + 4);
            } else {
                qraw[blk] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.q) + qrow + blk * 32 + g4 * 8);
            }
        }
    }
    const uint32_t L = split_length(a, b);
    const uint32_t tps = kWavesPerWg * cpw * kChunk;
    const uint32_t nsplit = (L + tps - 1) / tps;
    if (split >= nsplit) return;  // includes L == 0 (the combine kernel writes zeros)

    // ---- Q fragments (B operand of the QK MFMA): lane (g4, n) holds head n,
    // dims 32*blk + 8*g4 .. +7 of every block.  Codes enter the MFMA as fp16
    // (code + 1152) (see codes4_to_half_biased), so each block's dot carries an
    // extra 1152 * sum(q_blk); the accumulator starts at minus that amount.
    half8 qf[NB];
    half8 ql[kLo ? NB : 1];
    float kbias[NB];
    {
#pragma unroll
        for (uint32_t blk = 0; blk < NB; ++blk) {
            half8 v = {};
            half8 lo = {};
            float qs = 0.0f;
            if (n < G || (QPAIR && n >= 8 && n < 8 + G)) {
                if constexpr (QPAIR) {
                    // columns < G: hi parts; columns 8..8+G-1: lo parts of head n - 8
                    const float4 x0 = q32raw[blk][0];
                    const float4 x1 = q32raw[blk][1];
                    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const _Float16 hi = static_cast<_Float16>(xs[i]);
                        v[i] = n < 8 ? hi : static_cast<_Float16>(xs[i] - static_cast<float>(hi));
                        qs += static_cast<float>(v[i]);
                    }
                } else if constexpr (QF32) {
                    const float4 x0 = q32raw[blk][0];
                    const float4 x1 = q32raw[blk][1];
                    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const _Float16 hi = static_cast<_Float16>(xs[i]);
                        v[i] = hi;
                        lo[i] = static_cast<_Float16>(xs[i] - static_cast<float>(hi));
                        qs += static_cast<float>(hi) + static_cast<float>(lo[i]);
                    }
                } else {
                    v = __builtin_bit_cast(half8, qraw[QF32 ? 0 : blk]);
#pragma unroll
                    for (int i = 0; i < 8; ++i) qs += static_cast<float>(v[i]);
                }
            }
            qs = rows_reduce(qs, AddOp{});
            kbias[blk] = kCodeBias * qs;
            qf[blk] = v;
            if (kLo) ql[kLo ? blk : 0] = lo;
        }
    }

    float m_run = -INFINITY;
    float l_run = 0.0f;
    float4v O[NM];
    float4v vbias[kVBias ? NB : 1];  // column sums of the PV B operand per block (V code bias)
#pragma unroll
    for (uint32_t mt = 0; mt < NM; ++mt) O[mt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t blk = 0; blk < (kVBias ? NB : 1); ++blk) vbias[blk] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    const half4 ones = {(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};

    // With the fused append the splits cover the L-1 cached keys; the new token
    // (position L-1, whose cache slot may hold older bytes or be written meanwhile
    // by append_record: masked) has its own record.
    const uint32_t Lc = APPEND ? L - 1 : L;
    const uint32_t nsteps = (Lc + kChunk - 1) / kChunk;
    // Packed tokens: column n's context is shorter by the packed tokens after its own
    // (Lc_col); steps past Lc_lo, the shortest, mask per column.
    const uint32_t Lc_lo = Lc - (a.pack - 1);
    const uint32_t Lc_col = a.pack == 1 ? Lc : Lc - (a.pack - 1 - min(n, G - 1) / (G / a.pack));
    const uint32_t n_steps = first < nsteps ? min(n_max, (nsteps - first + stride - 1) / stride) : 0;
    // Per-wave LDS staging of one step's scales: [K: 32*NB][V: 32*NB] fp16.  Each lane
    // loads NB/2 scales (no redundancy) and re-reads the 4*NB it needs from LDS.
    uint16_t* s_sc = reinterpret_cast<uint16_t*>(smem + 32 * kWavesPerWg + kWavesPerWg * G * D) + wave * (2 * kChunk * NB);

    // A step that reaches past L (only the sequence's last) is masked under a
    // wave-uniform branch: its scores go to -inf and its V scales to 0 (the memory
    // past L may hold anything, including non-finite scales).
    auto compute_step = [&](uint32_t c, const Step& st) __attribute__((always_inline)) {
        const uint32_t tok0 = c * kChunk;
        const bool tail = tok0 + kChunk > Lc_lo;
        if constexpr (!KF16) *reinterpret_cast<ScaleVec*>(s_sc + lane * (NB / 2)) = st.ks;
        if constexpr (!VF16) {
            ScaleVec vsv = st.vs;
            if (tail && tok0 + lane / 2 >= Lc) vsv = ScaleVec{};
            *reinterpret_cast<ScaleVec*>(s_sc + kChunk * NB + lane * (NB / 2)) = vsv;
        }

        // ---- scores S^T[token][head], one MFMA per q8_0 block, block scale in fp32
        float s[2][4];
        if constexpr (KF16) {
            // fp16 keys: one accumulator chain over the blocks, no scale
#pragma unroll
            for (uint32_t J = 0; J < 2; ++J) {
                float4v c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (uint32_t cc = 0; cc < NC; ++cc) {
                    const half8 a0 = __builtin_bit_cast(half8, st.k[J][cc][0]);  // block 2cc
                    const half8 a1 = __builtin_bit_cast(half8, st.k[J][cc][KF16 ? 1 : 0]);  // block 2cc+1
                    c = mfma_16x16x32(a0, qf[2 * cc], c);
                    c = mfma_16x16x32(a1, qf[2 * cc + 1], c);
                    if (kLo) {
                        c = mfma_16x16x32(a0, ql[kLo ? 2 * cc : 0], c);
                        c = mfma_16x16x32(a1, ql[kLo ? 2 * cc + 1 : 0], c);
                    }
                }
                if constexpr (QPAIR) {
#pragma unroll
                    for (uint32_t i = 0; i < 4; ++i) c[i] += dpp_row_shl<8>(c[i]);  // + lo column
                }
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) s[J][i] = c[i] * a.scale_log2;
            }
        } else
#pragma unroll
        for (uint32_t J = 0; J < 2; ++J) {
            uint4 ksw[NB / 2];  // scales of tokens 16J + 4*g4 + i, all blocks
#pragma unroll
            for (uint32_t w = 0; w < NB / 2; ++w)
                ksw[w] = *reinterpret_cast<const uint4*>(s_sc + (16 * J + 4 * g4) * NB + w * 8);
            const uint16_t* ks16 = reinterpret_cast<const uint16_t*>(&ksw[0]);
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t cc = 0; cc < NC; ++cc) {
                const uint4 w = st.k[J][cc][0];
                const half8 a0 = codes8_to_half8_biased(w.x, w.y);  // block 2cc
                const half8 a1 = codes8_to_half8_biased(w.z, w.w);  // block 2cc+1
                const float b0 = -kbias[2 * cc], b1 = -kbias[2 * cc + 1];
                float4v c0 = mfma_16x16x32(a0, qf[2 * cc], float4v{b0, b0, b0, b0});
                float4v c1 = mfma_16x16x32(a1, qf[2 * cc + 1], float4v{b1, b1, b1, b1});
                if (kLo) {
                    c0 = mfma_16x16x32(a0, ql[kLo ? 2 * cc : 0], c0);
                    c1 = mfma_16x16x32(a1, ql[kLo ? 2 * cc + 1 : 0], c1);
                }
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    acc[i] = fmaf(c0[i], f16_bits_to_f32(ks16[i * NB + 2 * cc]), acc[i]);
                    acc[i] = fmaf(c1[i], f16_bits_to_f32(ks16[i * NB + 2 * cc + 1]), acc[i]);
                }
            }
            if constexpr (QPAIR) {
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) acc[i] += dpp_row_shl<8>(acc[i]);  // + lo column
            }
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                s[J][i] = acc[i] * a.scale_log2;
            }
        }

        if (tail) {
#pragma unroll
            for (uint32_t J = 0; J < 2; ++J)
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i)
                    if (tok0 + 16 * J + 4 * g4 + i >= Lc_col) s[J][i] = -INFINITY;
        }

        // ---- online softmax with a lazy running max: the accumulators are rescaled only
        // when a column's step max exceeds its running max by more than kRescaleSlack
        // (log2 units), so p <= 2^kRescaleSlack and p * scale stays inside fp16 range.
        float cmax = s[0][0];
#pragma unroll
        for (uint32_t J = 0; J < 2; ++J)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) cmax = fmaxf(cmax, s[J][i]);
        cmax = wave_max_xor_16_32(cmax);
        const bool grow = cmax > m_run + kRescaleSlack;
        if (__any(grow)) {
            const float m_new = grow ? cmax : m_run;
            const float alpha = grow ? fast_exp2(m_run - cmax) : 1.0f;  // (-inf - -inf would be NaN)
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (uint32_t mt = 0; mt < NM; ++mt) O[mt] *= alpha;
            if constexpr (kVBias) {
#pragma unroll
                for (uint32_t blk = 0; blk < NB; ++blk) vbias[blk] *= alpha;
            }
        }
        float psum = 0.0f;
        // a packed column may have no key yet (m_run = -inf): its p stay 0
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
#pragma unroll
        for (uint32_t J = 0; J < 2; ++J)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                s[J][i] = fast_exp2(s[J][i] - m_use);
                psum += s[J][i];
            }
        l_run += psum;

        // ---- O^T += V^T * (P^T scaled per block); V codes enter as (code + 1152), the
        // bias is removed at the end with the column sums accumulated in vbias.
        if constexpr (VF16) {
            // fp16 values: P^T unscaled; keys past the context are zeroed (the memory
            // there may hold non-finite values, and p = 0 would not cancel them)
#pragma unroll
            for (uint32_t J = 0; J < 2; ++J) {
                half4 pb;
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) pb[i] = static_cast<_Float16>(s[J][i]);
#pragma unroll
                for (uint32_t mt = 0; mt < NM; ++mt) {
                    const uint4 w = reinterpret_cast<const uint4&>(st.v[mt]);
                    half4 va = __builtin_bit_cast(half4, J == 0 ? make_uint2(w.x, w.y) : make_uint2(w.z, w.w));
                    if (tail) {
#pragma unroll
                        for (uint32_t i = 0; i < 4; ++i)
                            if (tok0 + 16 * J + 4 * g4 + i >= Lc) va[i] = static_cast<_Float16>(0.0f);
                    }
                    O[mt] = mfma_16x16x16(va, pb, O[mt]);
                }
            }
        } else
#pragma unroll
        for (uint32_t J = 0; J < 2; ++J) {
            uint4 vsw[NB / 2];
#pragma unroll
            for (uint32_t w = 0; w < NB / 2; ++w)
                vsw[w] = *reinterpret_cast<const uint4*>(s_sc + kChunk * NB + (16 * J + 4 * g4) * NB + w * 8);
            const uint16_t* vs16 = reinterpret_cast<const uint16_t*>(&vsw[0]);
#pragma unroll
            for (uint32_t blk = 0; blk < NB; ++blk) {
                half4 pb;
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    pb[i] = static_cast<_Float16>(s[J][i] * f16_bits_to_f32(vs16[i * NB + blk]));
                }
#pragma unroll
                for (uint32_t sub = 0; sub < 2; ++sub) {
                    const uint32_t mt = 2 * blk + sub;
                    const uint2 vw = reinterpret_cast<const uint2&>(st.v[mt]);
                    const uint32_t word = J == 0 ? vw.x : vw.y;
                    if constexpr (kVBias) O[mt] = mfma_16x16x16(codes4_to_half4_biased(word), pb, O[mt]);
                    else O[mt] = mfma_16x16x16(codes4_to_half4(word), pb, O[mt]);
                }
                if constexpr (kVBias) vbias[blk] = mfma_16x16x16(ones, pb, vbias[blk]);
            }
        }
    };

    // Software pipeline over the local steps [0, n_steps): while step i computes, the
    // loads of steps i+1 .. i+kRing-1 are in flight (fully unrolled so S[] stays in
    // registers).
    for (uint32_t i = 0; i < n_steps; i += kRing) {
#pragma unroll
        for (uint32_t r = 0; r < kRing; ++r) {
            if (i + r >= n_steps) break;
            if (i + r + kRing - 1 < n_steps) load_step(S[(r + kRing - 1) % kRing]);
            compute_step(first + (i + r) * stride, S[r]);
        }
    }
    if constexpr (kVBias) {
#pragma unroll
        for (uint32_t mt = 0; mt < NM; ++mt) O[mt] -= kCodeBias * vbias[mt / 2];
    }

    // ---- wave-level sums, then the cross-wave merge in LDS: each wave leaves its
    // state there (float4 per lane, a layout whose stores hit distinct banks), one
    // barrier, then every thread merges float4 slices of the record in wave order and
    // stores them (no second barrier: each thread derives the merge weights itself).
    l_run = rows_reduce(l_run, AddOp{});
    float* s_m = smem;                          // [waves][16]
    float* s_l = smem + 16 * kWavesPerWg;       // [waves][16]
    float4* s_O = reinterpret_cast<float4*>(smem + 32 * kWavesPerWg);  // [waves][NM][4 g4][G]
    if (g4 == 0) {
        s_m[wave * 16 + n] = m_run;
        s_l[wave * 16 + n] = l_run;
    }
    if (n < G) {
#pragma unroll
        for (uint32_t mt = 0; mt < NM; ++mt)
            s_O[((wave * NM + mt) * 4 + g4) * G + n] = make_float4(O[mt][0], O[mt][1], O[mt][2], O[mt][3]);
    }
    __syncthreads();

    // Partial record of one split: [O: G*D][m: G][l: G] padded to a multiple of 4 floats,
    // so every record starts 16-byte aligned.
    const uint32_t rec = record_floats(G, D);
    float* mine = a.part + ((static_cast<size_t>(b) * geo.kv_heads + h) * (a.max_splits + 1) + split) * rec;
    for (uint32_t c4 = tid; c4 < G * D / 4; c4 += blockDim.x) {
        const uint32_t hn = (4 * c4) / D, dim = (4 * c4) % D;
        const uint32_t mt = dim / 16, gq = (dim % 16) / 4;
        float mw[kWavesPerWg];
        float M = -INFINITY;
#pragma unroll
        for (uint32_t w = 0; w < kWavesPerWg; ++w) {
            mw[w] = s_m[w * 16 + hn];
            M = fmaxf(M, mw[w]);
        }
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float Ls = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < kWavesPerWg; ++w) {
            if (mw[w] == -INFINITY) continue;
            const float f = exp2_safe(mw[w] - M);
            const float4 v = s_O[((w * NM + mt) * 4 + gq) * G + hn];
            o.x += v.x * f;
            o.y += v.y * f;
            o.z += v.z * f;
            o.w += v.w * f;
            Ls += s_l[w * 16 + hn] * f;
        }
        *reinterpret_cast<float4*>(mine + 4 * c4) = o;
        if (dim == 0) {
            mine[G * D + hn] = M;
            mine[G * D + G + hn] = Ls;
        }
    }
}



// Workgroups of decode_kernel resident on the chip at its occupancy: 256 CUs x 4
// SIMDs x waves per SIMD, 4 waves per workgroup.
// f32: an fp32 query with separate lo fragments (more than 8 heads per kv head).
uint32_t resident_workgroups(uint32_t D, bool f32, uint32_t mode) {
    uint32_t wpe = D == 128 ? (f32 ? DecodeTuning<128, true>::waves_per_eu : DecodeTuning<128, false>::waves_per_eu)
                            : (f32 ? DecodeTuning<256, true>::waves_per_eu : DecodeTuning<256, false>::waves_per_eu);
    if (D == 256 && mode == MIIKV_KV_Q8_FP16) wpe = 1;
    return 256 * 4 * wpe / kWavesPerWg;
}

struct Plan {
    uint32_t cpw;
    bool adaptive;  // steps per wave chosen on the device (launch_cpw)
    uint32_t splits;
    uint64_t counter_bytes;
    uint64_t part_bytes;
};

// rowsets: row sets of one sequence (a suffix run as decodes), all of about the same
// length: the host plan is the launch's (no device-side choice), XCD-ordered.
Plan make_plan(const miikv_view* v, uint32_t q_heads, uint32_t batch, uint32_t max_context,
               uint32_t cpw_cap = 64, bool rowsets = false) {
    Plan p;
    const uint64_t chunks = (static_cast<uint64_t>(max_context) + kChunk - 1) / kChunk;
    const uint64_t waves = chunks * v->kv_heads * batch;
    // D = 256, one sequence: a wave holds one step in flight (its step buffer is
    // twice D = 128's), and one workgroup per CU with twice the steps per wave
    // measured faster than two (24q/4kv batch 1, µs: 16k 17.9 -> 16.7, 32k 24.1 ->
    // 23.0; 4k and 64k unchanged).  Batches keep the full target (config 3 is tuned so).
    const uint64_t target = (v->head_dim == 256 && batch == 1) ? kTargetWaves / 2 : kTargetWaves;
    uint64_t cpw = (waves + target - 1) / target;
    // A batch: cpw is the floor of the device-side choice (launch_cpw), which
    // can only raise it; the records and the grid are sized for the floor, a
    // quarter of the all-sequences-full value.
    if (batch > 1 && !rowsets) cpw = (cpw + 3) / 4;
    p.adaptive = batch > 1 && !rowsets;
    if (cpw < 1) cpw = 1;
    if (cpw > cpw_cap) cpw = cpw_cap;
    p.cpw = static_cast<uint32_t>(cpw);
    const uint64_t tps = kWavesPerWg * cpw * kChunk;
    p.splits = static_cast<uint32_t>((static_cast<uint64_t>(max_context) + tps - 1) / tps);
    if (p.splits == 0) p.splits = 1;
    const uint64_t G = q_heads / v->kv_heads;
    p.counter_bytes = 0;
    p.part_bytes = static_cast<uint64_t>(batch) * v->kv_heads * (p.splits + 1) * record_floats(G, v->head_dim) * 4;
    p.part_bytes = (p.part_bytes + 255) / 256 * 256;
    return p;
}

}  // namespace
}  // namespace miikv

using namespace miikv;

extern "C" uint64_t miikv_decode_workspace_bytes(const miikv_view* view, uint32_t q_heads, uint32_t batch,
                                                 uint32_t max_context) {
    if (validate_view(view) != MIIKV_OK || view->kv_heads == 0 || q_heads % view->kv_heads != 0 || batch == 0)
        return 0;
    if (q_heads / view->kv_heads > 16) return 0;  // the MFMA serves at most 16 query heads per kv head
    const Plan p = make_plan(view, q_heads, batch, max_context);
    return p.counter_bytes + p.part_bytes;
}

namespace {
__global__ void zero_kernel(uint4* p, uint64_t n16) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
        p[i] = make_uint4(0, 0, 0, 0);
}
}  // namespace

extern "C" miikv_status miikv_workspace_init(void* workspace, uint64_t bytes, void* stream) {
    if (workspace == nullptr || (bytes & 15u) != 0 || (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
        return MIIKV_EINVAL;
    if (bytes == 0) return MIIKV_OK;
    uint64_t blocks = (bytes / 16 + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(zero_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<uint4*>(workspace), bytes / 16);
    return hip_status(hipGetLastError());
}

#ifndef MIIKV_NARROW_COMBINE
#define MIIKV_NARROW_COMBINE 1
#endif
#ifndef MIIKV_NARROW_THREADS
#define MIIKV_NARROW_THREADS 16384
#endif
#ifndef MIIKV_ROWSET_MAX_CPW
#define MIIKV_ROWSET_MAX_CPW 32
#endif
constexpr uint32_t kRowsetMaxCpw = MIIKV_ROWSET_MAX_CPW;
// Columns a row set of an fp32 query may fill: 8 keeps its lo parts in the spare
// columns (decode_kernel's QPAIR form); 16 packs twice the tokens with a second
// fragment set.
#ifndef MIIKV_ROWSET_COLS_F32
#define MIIKV_ROWSET_COLS_F32 8
#endif
constexpr uint32_t kRowsetColsF32 = MIIKV_ROWSET_COLS_F32;
#ifndef MIIKV_DECODE_QPAIR
#define MIIKV_DECODE_QPAIR 1
#endif
namespace {
template <uint32_t D, bool F32, bool APP, bool KF, bool VF>
void launch_decode_t(dim3 grid, size_t lds, hipStream_t s, const SplitArgs& a) {
    // An fp32 query of up to 8 heads per kv head pairs its lo parts into the spare columns
    // (at D = 256 the second fragment set would cost occupancy; at D = 128 it doubles the
    // score MFMAs).  Row sets of one sequence over q8 planes load through the L2.
    const bool pair = F32 && a.group <= 8 && MIIKV_DECODE_QPAIR;
    if constexpr (!APP && !KF && !VF) {
        if (a.rowset_order) {
            if (pair)
                hipLaunchKernelGGL((decode_kernel<D, F32, false, false, false, F32, true>), grid, dim3(64 * kWavesPerWg),
                                   lds, s, a);
            else
                hipLaunchKernelGGL((decode_kernel<D, F32, false, false, false, false, true>), grid,
                                   dim3(64 * kWavesPerWg), lds, s, a);
            return;
        }
    }
    if (pair)
        hipLaunchKernelGGL((decode_kernel<D, F32, APP, KF, VF, F32>), grid, dim3(64 * kWavesPerWg), lds, s, a);
    else
        hipLaunchKernelGGL((decode_kernel<D, F32, APP, KF, VF, false>), grid, dim3(64 * kWavesPerWg), lds, s, a);
}
// Runtime flags -> kernel instance.  The fused append exists for q8 planes only (the
// caller has rejected it for the other modes).
template <uint32_t D>
void launch_decode(bool f32, bool app, bool kf, bool vf, dim3 grid, size_t lds, hipStream_t s, const SplitArgs& a) {
    if (app) {
        if (f32) launch_decode_t<D, true, true, false, false>(grid, lds, s, a);
        else launch_decode_t<D, false, true, false, false>(grid, lds, s, a);
        return;
    }
    if (f32) {
        if (kf && vf) launch_decode_t<D, true, false, true, true>(grid, lds, s, a);
        else if (kf) launch_decode_t<D, true, false, true, false>(grid, lds, s, a);
        else if (vf) launch_decode_t<D, true, false, false, true>(grid, lds, s, a);
        else launch_decode_t<D, true, false, false, false>(grid, lds, s, a);
    } else {
        if (kf && vf) launch_decode_t<D, false, false, true, true>(grid, lds, s, a);
        else if (kf) launch_decode_t<D, false, false, true, false>(grid, lds, s, a);
        else if (vf) launch_decode_t<D, false, false, false, true>(grid, lds, s, a);
        else launch_decode_t<D, false, false, false, false>(grid, lds, s, a);
    }
}
}  // namespace

// The new token's rows of a fused append + decode: fp16 rows, or fp32 rows with the
// reference's K prologue (k_norm_weight set) or without it.
struct NewRows {
    const uint16_t* k16 = nullptr;
    const uint16_t* v16 = nullptr;
    const float* k32 = nullptr;
    const float* v32 = nullptr;
    const float* k_norm_weight = nullptr;
    float theta = 0.0f;
    float epsilon = 0.0f;
    bool any() const { return k16 != nullptr || k32 != nullptr; }
};

// Dynamic LDS of decode_kernel with G columns: each wave's (m, l) and O^T for the
// cross-wave merge, and its scale staging.
static size_t decode_lds_bytes(uint32_t G, uint32_t D) {
    return (32 * kWavesPerWg + kWavesPerWg * G * D) * sizeof(float) + kWavesPerWg * 2 * kChunk * (D / 32) * sizeof(uint16_t);
}

// Row sets that all read one sequence (a short suffix run as a batch of decodes):
// row set b has context length (len_ptr ? *len_ptr : 0) + len_add + b, and row sets
// at or past *count_ptr (when set) are skipped.
struct RowSets {
    const uint32_t* len_ptr;
    uint32_t len_add;
    const uint32_t* count_ptr;
    uint32_t seq;
    uint32_t pack;  // tokens per row set (divides batch; no count_ptr when > 1)
};

static miikv_status decode_impl(const miikv_view* view, const NewRows& rows,
                                const void* q, uint32_t q_dtype, uint32_t q_heads, float scale, uint32_t batch,
                                const uint32_t* d_lengths, const miikv_decode_state* decode_state,
                                uint32_t max_context, float* out, const float* gate, float* gated_out,
                                void* gated_q8_1, void* workspace, uint64_t workspace_bytes, void* stream,
                                const RowSets* rs = nullptr) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (q == nullptr || batch == 0 || q_heads == 0 || q_heads % view->kv_heads != 0 || !std::isfinite(scale))
        return MIIKV_EINVAL;
    // packed tokens: batch / pack row sets of pack * G columns
    const uint32_t pack = rs != nullptr ? rs->pack : 1u;
    if (pack == 0 || batch % pack != 0 || (pack > 1 && rs->count_ptr != nullptr)) return MIIKV_EINVAL;
    batch /= pack;
    const uint32_t G = q_heads / view->kv_heads * pack;
    if (G > 16) return MIIKV_EUNSUPPORTED;
    if (q_dtype != MIIKV_DTYPE_F16 && q_dtype != MIIKV_DTYPE_F32) return MIIKV_EINVAL;
    if (out == nullptr && !(gate != nullptr && (gated_out != nullptr || gated_q8_1 != nullptr)))
        return MIIKV_EINVAL;
    if (gate == nullptr && (gated_out != nullptr || gated_q8_1 != nullptr)) return MIIKV_EINVAL;
    if (gate != nullptr && gated_out == nullptr && gated_q8_1 == nullptr) return MIIKV_EINVAL;
    if (rs == nullptr && d_lengths == nullptr && (decode_state == nullptr || batch != 1)) return MIIKV_EINVAL;
    if (max_context == 0 || max_context > view_seq_capacity(view)) return MIIKV_EINVAL;
    if (rs == nullptr && view->layout == MIIKV_LAYOUT_CONTIGUOUS && batch != 1) return MIIKV_EINVAL;
    // the fused append stores q8 rows
    if (rows.any() && view->quant_mode != MIIKV_KV_Q8_Q8) return MIIKV_EUNSUPPORTED;
    if (rows.k_norm_weight != nullptr && (!std::isfinite(rows.theta) || !std::isfinite(rows.epsilon)))
        return MIIKV_EINVAL;
    const Plan p = make_plan(view, q_heads * pack, batch, max_context, rs != nullptr ? kRowsetMaxCpw : 64u,
                             rs != nullptr);
    if (workspace == nullptr || workspace_bytes < p.counter_bytes + p.part_bytes) return MIIKV_EWORKSPACE;
    if (p.splits > 65535u || batch > 65535u || static_cast<uint64_t>(batch) * view->kv_heads > 0x7fffffffu)
        return MIIKV_EINVAL;

    SplitArgs a{};
    a.g = make_geo(*view);
    a.q = q;
    a.q_heads = q_heads;
    a.group = G;
    a.pack = pack;
    a.scale_log2 = scale * kLog2e;
    a.len_bstep = 0;
    a.count_ptr = nullptr;
    // Row sets of one sequence all read the same keys: with long items the workgroups
    // running at once stream the same addresses together, so the row-set route caps
    // the steps per wave lower (host plan and device choice alike: the records are
    // sized for the host's floor; exact suffix route at config 4: 1372 us at 64,
    // 1000 at 32, 1055 at 16); decode batches of distinct sequences keep 64.
    a.max_cpw = rs != nullptr ? kRowsetMaxCpw : 64u;
    a.rowset_order = rs != nullptr ? 1u : 0u;
    if (rs != nullptr) {  // row set b: len_add + b * pack (its last token's context)
        a.len_ptr = rs->len_ptr;
        a.len_stride = 0;
        a.len_add = rs->len_add + (pack - 1);
        a.len_bstep = pack;
        a.count_ptr = rs->count_ptr;
        if (view->layout == MIIKV_LAYOUT_PAGED) {  // every row set reads table row seq
            a.g.table = view->block_table + static_cast<size_t>(rs->seq) * view->table_stride;
            a.g.table_stride = 0;
        }
    } else if (d_lengths != nullptr) {
        a.len_ptr = d_lengths;
        a.len_stride = 1;
        a.len_add = 0;
    } else {
        a.len_ptr = &decode_state->position;
        a.len_stride = 0;
        a.len_add = 1;
    }
    a.max_context = max_context;
    a.cpw = p.cpw;
    a.max_splits = p.splits;
    a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + p.counter_bytes);
    a.out = out;
    a.gate = gate;
    a.gated_out = gated_out;
    a.gated_q8_1 = static_cast<uint8_t*>(gated_q8_1);
    a.k_new = rows.k16;
    a.v_new = rows.v16;
    a.k_new32 = rows.k32;
    a.v_new32 = rows.v32;
    a.k_norm_weight = rows.k_norm_weight;
    a.rope_step = rows.k_norm_weight != nullptr ? powf(rows.theta, -2.0f / 64.0f) : 0.0f;
    a.epsilon = rows.epsilon;
    a.q_f32 = q_dtype == MIIKV_DTYPE_F32;

    const size_t lds = decode_lds_bytes(G, view->head_dim);
    if (lds > 64 * 1024) return MIIKV_EUNSUPPORTED;
    // One workgroup per possible (sequence, kv head, split) work item, plus one per
    // (sequence, kv head) for the new token of the fused append.
    uint64_t wgs = static_cast<uint64_t>(p.splits) * view->kv_heads * batch +
                   (rows.any() ? static_cast<uint64_t>(view->kv_heads) * batch : 0);
    if (rs != nullptr) wgs = (wgs + 7) / 8 * 8;  // XCD-ordered items: a whole number of rounds over the XCDs
    if (wgs > 0x7fffffffu) return MIIKV_EINVAL;
    a.batch = batch;
    a.slots = p.adaptive ? resident_workgroups(view->head_dim, q_dtype == MIIKV_DTYPE_F32 && (view->head_dim == 128 || 2 * G > 16), view->quant_mode) : 0u;
    const dim3 grid(static_cast<uint32_t>(wgs));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool f32 = q_dtype == MIIKV_DTYPE_F32;
    // combine: one workgroup per (sequence, kv head, 32 output elements), or one thread
    // per 4 output elements when a row set holds at most kNarrowRecords records or the
    // launch has threads enough that way (config 2's single sequence: 1024 threads
    // for 65 records each, which the wide form reads in one round trip)
    const dim3 cgrid(batch * view->kv_heads, G * view->head_dim / 32);
    const uint64_t nthreads = static_cast<uint64_t>(batch) * view->kv_heads * G * view->head_dim / 4;
    const bool narrow = (p.splits + 1 <= kNarrowRecords || nthreads >= MIIKV_NARROW_THREADS) && MIIKV_NARROW_COMBINE;
    const dim3 ngrid(static_cast<uint32_t>((nthreads + 255) / 256));
    const bool app = rows.any();
    const bool kf = mode_k_f16(view->quant_mode), vf = mode_v_f16(view->quant_mode);
    if (view->head_dim == 128) {
        launch_decode<128>(f32, app, kf, vf, grid, lds, s, a);
        if (narrow && app) hipLaunchKernelGGL((combine_narrow_kernel<128, true>), ngrid, dim3(256), 0, s, a);
        else if (narrow) hipLaunchKernelGGL((combine_narrow_kernel<128, false>), ngrid, dim3(256), 0, s, a);
        else if (app) hipLaunchKernelGGL((combine_kernel<128, true>), cgrid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((combine_kernel<128, false>), cgrid, dim3(256), 0, s, a);
    } else {
        launch_decode<256>(f32, app, kf, vf, grid, lds, s, a);
        if (narrow && app) hipLaunchKernelGGL((combine_narrow_kernel<256, true>), ngrid, dim3(256), 0, s, a);
        else if (narrow) hipLaunchKernelGGL((combine_narrow_kernel<256, false>), ngrid, dim3(256), 0, s, a);
        else if (app) hipLaunchKernelGGL((combine_kernel<256, true>), cgrid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((combine_kernel<256, false>), cgrid, dim3(256), 0, s, a);
    }
    return hip_status(hipGetLastError());
}

namespace miikv {
// Suffix attention of a short suffix as a batch of decodes over one sequence: token t
// is row set t with context P + t + 1 (the cache already holds the suffix's rows).
// Each row set streams its context once, so this pays for few tokens only; it
// serves miikv_suffix_attn below a token-count threshold (miikv_suffix.hip).
// Tokens per row set: the largest divisor of token_count whose columns (tokens x
// query heads per kv head) fit the 16 of the MFMA and the kernel's LDS; with a device
// token count, 1.
bool decode_columns_fit(uint32_t G, uint32_t D) { return G <= 16 && decode_lds_bytes(G, D) <= 64 * 1024; }

// max_cols: 16 (the MFMA's columns), or 8 for an fp32 query, whose lo parts then ride
// in the other 8 columns (one MFMA per block at the fp16-query register budget).
uint32_t suffix_pack(const miikv_view* view, uint32_t q_heads, uint32_t token_count, bool device_count,
                     uint32_t max_cols) {
    const uint32_t G = q_heads / view->kv_heads;
    if (device_count || G == 0 || G > 16) return 1;
    for (uint32_t p = std::min<uint32_t>(max_cols / G, token_count); p > 1; --p)
        if (token_count % p == 0 && decode_lds_bytes(p * G, view->head_dim) <= 64 * 1024) return p;
    return 1;
}

uint64_t suffix_by_decode_bytes(const miikv_view* view, uint32_t q_heads, uint32_t token_count, uint32_t bound) {
    // the largest of the packed plans (fp16 and fp32 queries, host token count) and the
    // unpacked one (device count)
    uint64_t most = 0;
    for (const uint32_t pk : {1u, suffix_pack(view, q_heads, token_count, false, 16),
                              suffix_pack(view, q_heads, token_count, false, kRowsetColsF32)}) {
        const Plan p = make_plan(view, q_heads * pk, token_count / pk, bound, kRowsetMaxCpw, true);
        most = std::max(most, p.counter_bytes + p.part_bytes);
    }
    return most;
}

miikv_status suffix_by_decode(const miikv_view* view, const void* q, uint32_t q_dtype, uint32_t q_heads, float scale,
                              uint32_t token_count, uint32_t base_position, uint32_t seq,
                              const miikv_prefill_state* prefill_state, uint32_t bound, float* out, const float* gate,
                              float* gated_out, void* workspace, uint64_t workspace_bytes, void* stream) {
    RowSets rs;
    rs.len_ptr = prefill_state ? &prefill_state->base_position : nullptr;
    rs.len_add = prefill_state ? 1u : base_position + 1u;
    rs.count_ptr = prefill_state ? &prefill_state->token_count : nullptr;
    rs.seq = seq;
    // An fp32 query of 4..16 tokens fills 8 columns per row set, its lo parts in the
    // other 8 (more row sets at two waves per SIMD: config 4 shape, T = 4 / 8: 26.5 /
    // 31.7 -> 20.4 / 26.1 us); fewer or more tokens pack 16 columns with a second
    // fragment set (T = 2: 16.6 against 17.2 us; the exact route at T = 512: 790
    // against 963 us, where twice the row sets' operand conversions cost more).
    const bool pair_cols = q_dtype == MIIKV_DTYPE_F32 && token_count >= 4 && token_count <= 16;
    rs.pack = suffix_pack(view, q_heads, token_count, prefill_state != nullptr, pair_cols ? kRowsetColsF32 : 16u);
    return decode_impl(view, NewRows{}, q, q_dtype, q_heads, scale, token_count, nullptr, nullptr, bound, out, gate,
                       gated_out, nullptr, workspace, workspace_bytes, stream, &rs);
}
}  // namespace miikv

extern "C" miikv_status miikv_decode_attn_q8_1(const miikv_view* view, const void* q, uint32_t q_dtype,
                                               uint32_t q_heads, float scale, uint32_t batch,
                                               const uint32_t* d_lengths, const miikv_decode_state* decode_state,
                                               uint32_t max_context, float* out, const float* gate,
                                               float* gated_out, void* gated_q8_1, void* workspace,
                                               uint64_t workspace_bytes, void* stream) {
    return decode_impl(view, NewRows{}, q, q_dtype, q_heads, scale, batch, d_lengths, decode_state, max_context,
                       out, gate, gated_out, gated_q8_1, workspace, workspace_bytes, stream);
}

extern "C" miikv_status miikv_decode_attn(const miikv_view* view, const void* q, uint32_t q_dtype, uint32_t q_heads,
                                          float scale, uint32_t batch, const uint32_t* d_lengths,
                                          const miikv_decode_state* decode_state, uint32_t max_context, float* out,
                                          const float* gate, float* gated_out, void* workspace,
                                          uint64_t workspace_bytes, void* stream) {
    return decode_impl(view, NewRows{}, q, q_dtype, q_heads, scale, batch, d_lengths, decode_state, max_context,
                       out, gate, gated_out, nullptr, workspace, workspace_bytes, stream);
}

extern "C" miikv_status miikv_decode_append_attn(const miikv_view* view, const uint16_t* k_new,
                                                 const uint16_t* v_new, const void* q, uint32_t q_dtype,
                                                 uint32_t q_heads, float scale, uint32_t batch,
                                                 const uint32_t* d_lengths, const miikv_decode_state* decode_state,
                                                 uint32_t max_context, float* out, const float* gate,
                                                 float* gated_out, void* gated_q8_1, void* workspace,
                                                 uint64_t workspace_bytes, void* stream) {
    if (k_new == nullptr || v_new == nullptr) return MIIKV_EINVAL;
    NewRows rows;
    rows.k16 = k_new;
    rows.v16 = v_new;
    return decode_impl(view, rows, q, q_dtype, q_heads, scale, batch, d_lengths, decode_state, max_context,
                       out, gate, gated_out, gated_q8_1, workspace, workspace_bytes, stream);
}


extern "C" miikv_status miikv_decode_append_attn_f32(const miikv_view* view, const float* k_new, const float* v_new,
                                                     const float* k_norm_weight, float theta, float epsilon,
                                                     const void* q, uint32_t q_dtype, uint32_t q_heads, float scale,
                                                     uint32_t batch, const uint32_t* d_lengths,
                                                     const miikv_decode_state* decode_state, uint32_t max_context,
                                                     float* out, const float* gate, float* gated_out,
                                                     void* gated_q8_1, void* workspace, uint64_t workspace_bytes,
                                                     void* stream) {
    if (k_new == nullptr || v_new == nullptr) return MIIKV_EINVAL;
    if (k_norm_weight != nullptr && view != nullptr && view->head_dim < 64) return MIIKV_EINVAL;
    NewRows rows;
    rows.k32 = k_new;
    rows.v32 = v_new;
    rows.k_norm_weight = k_norm_weight;
    rows.theta = theta;
    rows.epsilon = epsilon;
    return decode_impl(view, rows, q, q_dtype, q_heads, scale, batch, d_lengths, decode_state, max_context, out,
                       gate, gated_out, gated_q8_1, workspace, workspace_bytes, stream);
}

// ---- decode without a caller workspace ---------------------------------------
// The split records live in a file-scope device array instead of a caller
// workspace.  Every GPU the library runs on holds its own copy until the process
// ends; host code uses its per-device address from hipGetSymbolAddress, never the
// array's name (a host-side stand-in that is not a device address).
// Calls are ordered on the GPU: one host lock covers each call's enqueue, and a
// call on another stream than the previous call's first waits for an event the
// previous call recorded after its kernels (both made once per device, at the first
// call).  Inside a stream capture neither the wait nor the record is issued: the
// graph's own order applies, and replays of such graphs on several streams at once
// race on the array.
namespace {
constexpr uint64_t kScratchBytes = 16ull << 20;
__device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
struct ScratchDevice {
    void* ptr = nullptr;          // the device address of `scratch`
    hipEvent_t done = nullptr;    // recorded after the last uncaptured call's kernels
    hipStream_t stream = nullptr; // that call's stream
    bool recorded = false;
};
ScratchDevice g_scratch[kMaxDevices];
std::mutex g_scratch_mutex;

// This device's scratch state, set up once per device (with that device current);
// the caller holds g_scratch_mutex.  Returns a status.
int scratch_for_current_device(ScratchDevice** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= kMaxDevices) return MIIKV_EUNSUPPORTED;
    ScratchDevice& sd = g_scratch[dev];
    if (sd.ptr == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e);
        if (ptr == nullptr) return MIIKV_EUNSUPPORTED;
        e = hipEventCreateWithFlags(&sd.done, hipEventDisableTiming);
        if (e != hipSuccess) return hip_status(e);
        sd.ptr = ptr;
    }
    *out = &sd;
    return MIIKV_OK;
}
}  // namespace

extern "C" uint64_t miikv_decode_scratch_max_bytes(void) { return kScratchBytes; }

extern "C" miikv_status miikv_decode_append_attn_noalloc(const miikv_view* view, const uint16_t* k_new,
                                                         const uint16_t* v_new, const void* q, uint32_t q_dtype,
                                                         uint32_t q_heads, float scale, uint32_t batch,
                                                         const uint32_t* d_lengths,
                                                         const miikv_decode_state* decode_state,
                                                         uint32_t max_context, float* out, const float* gate,
                                                         float* gated_out, void* gated_q8_1, void* stream) {
    if (k_new == nullptr || v_new == nullptr) return MIIKV_EINVAL;
    const uint64_t need = miikv_decode_workspace_bytes(view, q_heads, batch, max_context);
    if (need == 0) return MIIKV_EINVAL;
    if (need > kScratchBytes) return MIIKV_EWORKSPACE;  // beyond the fixed scratch: use miikv_decode_append_attn
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ScratchDevice* sd = nullptr;
    const int st = scratch_for_current_device(&sd);
    if (st != MIIKV_OK) return st;
    hipStream_t hs = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(hs, &cap);
    if (e != hipSuccess) return hip_status(e);
    const bool capturing = cap != hipStreamCaptureStatusNone;
    if (!capturing && sd->recorded && sd->stream != hs) {
        e = hipStreamWaitEvent(hs, sd->done, 0);
        if (e != hipSuccess) return hip_status(e);
    }
    NewRows rows;
    rows.k16 = k_new;
    rows.v16 = v_new;
    const miikv_status ds = decode_impl(view, rows, q, q_dtype, q_heads, scale, batch, d_lengths, decode_state,
                                        max_context, out, gate, gated_out, gated_q8_1, sd->ptr, kScratchBytes,
                                        stream);
    if (ds != MIIKV_OK || capturing) return ds;
    e = hipEventRecord(sd->done, hs);
    if (e != hipSuccess) return hip_status(e);
    sd->stream = hs;
    sd->recorded = true;
    return MIIKV_OK;
}
