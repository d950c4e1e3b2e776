// q8_0 append, canonical export/import, page copy, segment copy and state clone.
#include "miikv_common.hpp"

#include <cmath>
#include <cstdlib>

namespace miikv {

// Host-side validation of a view (shared with the decode launcher).
int validate_view(const miikv_view* v) {
    if (v == nullptr) return MIIKV_EINVAL;
    if (v->quant_mode > MIIKV_KV_Q8_Q8) return MIIKV_EINVAL;
    // q8 planes need their scales; fp16 planes have none
    if (v->k_codes == nullptr || v->v_codes == nullptr || (!mode_k_f16(v->quant_mode) && v->k_scales == nullptr) ||
        (!mode_v_f16(v->quant_mode) && v->v_scales == nullptr))
        return MIIKV_EINVAL;
    if (v->head_dim != 128 && v->head_dim != 256) return MIIKV_EUNSUPPORTED;
    if (v->kv_heads == 0 || v->page_tokens == 0 || v->page_tokens % 64 != 0) return MIIKV_EINVAL;
    if (v->layout == MIIKV_LAYOUT_CONTIGUOUS) {
        if (v->num_pages != 1) return MIIKV_EINVAL;
    } else if (v->layout == MIIKV_LAYOUT_PAGED) {
        if (v->block_table == nullptr || v->table_stride == 0 || v->num_pages == 0) return MIIKV_EINVAL;
    } else {
        return MIIKV_EINVAL;
    }
    return MIIKV_OK;
}

// Largest logical token count a sequence of this view can hold.
uint64_t view_seq_capacity(const miikv_view* v) {
    if (v->layout == MIIKV_LAYOUT_CONTIGUOUS) return v->page_tokens;
    return static_cast<uint64_t>(v->table_stride) * v->page_tokens;
}

namespace {

// Row inputs of the append kernel: fp16 rows, or fp32 rows with the optional K
// prologue of the reference store kernel (RMSNorm * weight, RoPE on dims 0..63).
struct AppendIn {
    const void* k;
    const void* v;
    const float* k_norm_weight;  // fp32 input only; null: no prologue
    float rope_step;             // theta^(-2/64), computed once on the host
    float epsilon;
};

__device__ __forceinline__ void load16_f32(const float* p, float (&x)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 f = *reinterpret_cast<const float4*>(p + 4 * i);
        x[4 * i] = f.x;
        x[4 * i + 1] = f.y;
        x[4 * i + 2] = f.z;
        x[4 * i + 3] = f.w;
    }
}

// K prologue on one lane's 16 dims d0 = 16*q16 ..: RMSNorm * weight, then RoPE on
// dims 0..63 (gfx906/kernels/qwen3_primitives.hip:7257-7281, 622-659).
// The sum of squares follows the reference's 256-lane LDS tree exactly: element t
// first meets t + D/2 (lanes q16 and q16 ^ groups/2), then t + D/4, ... down to the
// lane's own 16 values, pairs 8, 4, 2, 1 apart.  r = 1 / sqrt(ss / D + eps) with the
// correctly rounded square root and division (the reference's rsqrtf is the
// hardware approximation, within one ulp of it), value * r * weight in that order.
// RoPE pairs (i, i+32), i < 32, sit in lanes q16 and q16 ^ 2; pair i's angle is
// position * step^i, accumulated by repeated fp32 multiplication as the reference
// does, with step = theta^(-2/64) computed once on the host (one powf for every
// kernel, so the angles are the ones a host computes), and rotated with rope_sincos
// (the reference calls cosf and sinf).  No contraction into fused multiply-adds: every
// product and sum rounds as written, as in the oracle.
__device__ __forceinline__ void k_norm_rope16(float (&x)[16], const float* w, uint32_t q16, uint32_t groups,
                                              uint32_t D, uint32_t position, float step, float eps) {
#pragma clang fp contract(off)
    float sq[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sq[i] = x[i] * x[i];
    for (uint32_t o = groups / 2; o > 0; o >>= 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sq[i] += __shfl_xor(sq[i], o, 64);
    }
#pragma unroll
    for (int s2 = 8; s2 > 0; s2 >>= 1)
#pragma unroll
        for (int i = 0; i < s2; ++i) sq[i] += sq[i + s2];
    const float r = 1.0f / sqrtf(sq[0] / static_cast<float>(D) + eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 wv = *reinterpret_cast<const float4*>(w + 16 * q16 + 4 * i);
        x[4 * i] = x[4 * i] * r * wv.x;
        x[4 * i + 1] = x[4 * i + 1] * r * wv.y;
        x[4 * i + 2] = x[4 * i + 2] * r * wv.z;
        x[4 * i + 3] = x[4 * i + 3] * r * wv.w;
    }
    float partner[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) partner[i] = dpp_mov<0x4E>(x[i]);  // lane ^ 2
    if (q16 >= 4) return;
    float angle = static_cast<float>(position);
    // first pair index of this lane: 0, or 16 (step applied 16 times, in order)
#pragma unroll
    for (uint32_t i = 0; i < 16; ++i) {
        const float next = angle * step;
        angle = (q16 & 1) ? next : angle;
    }
    const bool low = q16 < 2;           // dims i (low) or i + 32 (high) of the pairs
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        float sn, cs;
        rope_sincos(angle, &sn, &cs);
        if (low) x[j] = x[j] * cs - partner[j] * sn;
        else x[j] = partner[j] * sn + x[j] * cs;
        angle *= step;
    }
}

// Eight values -> eight fp16 (round to nearest even) in one 16-byte word.
__device__ __forceinline__ uint4 pack8_f16(const float* x) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = static_cast<uint32_t>(f32_to_f16_bits(x[2 * i])) | (static_cast<uint32_t>(f32_to_f16_bits(x[2 * i + 1])) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// One thread per (row, 16-dim group); a row is (token, kv_head).  Adjacent
// lanes (2i, 2i+1) hold the two halves of one 32-value block, and the D/16
// lanes of a row are consecutive.
template <bool F32>
__global__ void __launch_bounds__(256) append_kernel(
    Geo g, AppendIn in, uint32_t token_count, uint32_t base_position, uint32_t seq,
    const miikv_prefill_state* __restrict__ ps, const miikv_decode_state* __restrict__ ds,
    const uint32_t* __restrict__ positions) {
    if (ps != nullptr) {
        base_position = ps->base_position;
        token_count = min(token_count, ps->token_count);
    } else if (ds != nullptr) {
        base_position = ds->position;
        token_count = 1;
    }
    const uint32_t D = g.head_dim;
    const uint32_t groups = D / 16;
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t row = gid / groups;
    const uint32_t q16 = static_cast<uint32_t>(gid % groups);
    const uint32_t token = static_cast<uint32_t>(row / g.kv_heads);
    const uint32_t head = static_cast<uint32_t>(row % g.kv_heads);
    if (token >= token_count) return;  // whole rows exit together

    uint32_t pos;
    if (positions != nullptr) {  // batched decode: row `token` is sequence `token`
        seq = token;
        pos = positions[token];
    } else {
        pos = base_position + token;
    }
    const uint64_t limit = (g.layout == MIIKV_LAYOUT_PAGED)
                               ? static_cast<uint64_t>(g.table_stride) * g.page_tokens
                               : g.page_tokens;
    const bool in_range = pos < limit;

    const size_t src = static_cast<size_t>(row) * D + q16 * 16;
    float xk[16], xv[16];
    if constexpr (F32) {
        load16_f32(static_cast<const float*>(in.k) + src, xk);
        load16_f32(static_cast<const float*>(in.v) + src, xv);
        if (in.k_norm_weight != nullptr)
            k_norm_rope16(xk, in.k_norm_weight, q16, groups, D, pos, in.rope_step, in.epsilon);
    } else {
        load16_f16(static_cast<const uint16_t*>(in.k) + src, xk);
        load16_f16(static_cast<const uint16_t*>(in.v) + src, xv);
    }
    int8_t qk[16], qv[16];
    float sk, sv;
    quantize16(xk, qk, sk);  // both lanes of the pair reach the shuffles
    quantize16(xv, qv, sv);
    if (!in_range) return;

    const size_t slab = slab_of(g, seq, pos, head);
    const uint32_t tp = pos % g.page_tokens;
    const size_t slab_bytes = static_cast<size_t>(g.page_tokens) * D;
    const uint32_t d0 = q16 * 16;

    // K: dims d0..d0+7 and d0+8..d0+15 are two 8-element runs of the tiled layout.
    if (g.k_f16) {
        uint16_t* kslab = reinterpret_cast<uint16_t*>(g.k_codes) + slab * slab_bytes;
        *reinterpret_cast<uint4*>(kslab + k_code_offset(tp, d0, D)) = pack8_f16(xk);
        *reinterpret_cast<uint4*>(kslab + k_code_offset(tp, d0 + 8, D)) = pack8_f16(xk + 8);
    } else {
        int8_t* kslab = g.k_codes + slab * slab_bytes;
        uint32_t packed[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            packed[w] = (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * w]))) |
                        (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * w + 1])) << 8) |
                        (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * w + 2])) << 16) |
                        (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * w + 3])) << 24);
        }
        *reinterpret_cast<uint2*>(kslab + k_code_offset(tp, d0, D)) = make_uint2(packed[0], packed[1]);
        *reinterpret_cast<uint2*>(kslab + k_code_offset(tp, d0 + 8, D)) = make_uint2(packed[2], packed[3]);
    }

    // V: each dim is its own token-contiguous run; one element per dim.
    if (g.v_f16) {
        uint16_t* vslab = reinterpret_cast<uint16_t*>(g.v_codes) + slab * slab_bytes;
#pragma unroll
        for (int i = 0; i < 16; ++i) vslab[v_code_offset(tp, d0 + i, D)] = f32_to_f16_bits(xv[i]);
    } else {
        int8_t* vslab = g.v_codes + slab * slab_bytes;
#pragma unroll
        for (int i = 0; i < 16; ++i) vslab[v_code_offset(tp, d0 + i, D)] = qv[i];
    }

    if ((q16 & 1) == 0) {
        const size_t sidx = (slab * g.page_tokens + tp) * (D / 32) + d0 / 32;
        if (!g.k_f16) g.k_scales[sidx] = f32_to_f16_bits(sk);
        if (!g.v_f16) g.v_scales[sidx] = f32_to_f16_bits(sv);
    }
}

// Bulk append of whole 32-token groups: one workgroup per (group, kv head), one
// thread per (token, 16-dim group) with the same arithmetic as append_kernel (so the
// codes are identical), but the codes and scales are assembled in LDS and leave as
// contiguous 16-byte stores: a 32-token group owns 32*D contiguous bytes of the K
// slab (two 16-token tiles), 32*D of the V slab (one group) and 32*D/32 scales of
// each kind.  base_position is a multiple of 32 and every group lies inside the
// sequence's capacity (checked on the host).
template <bool F32>
__global__ void __launch_bounds__(512) append_tile_kernel(Geo g, AppendIn in, uint32_t base_position,
                                                          uint32_t seq) {
    extern __shared__ uint4 s_tile[];
    const uint32_t D = g.head_dim;
    const uint32_t groups = D / 16;
    const uint32_t head = blockIdx.y;
    const uint32_t tl = threadIdx.x / groups;  // token within the 32-token group
    const uint32_t q16 = threadIdx.x % groups;
    const uint32_t token = blockIdx.x * 32 + tl;
    const uint32_t pos = base_position + token;
    const size_t src = (static_cast<size_t>(token) * g.kv_heads + head) * D + q16 * 16;
    float xk[16], xv[16];
    if constexpr (F32) {
        load16_f32(static_cast<const float*>(in.k) + src, xk);
        load16_f32(static_cast<const float*>(in.v) + src, xv);
        if (in.k_norm_weight != nullptr)
            k_norm_rope16(xk, in.k_norm_weight, q16, groups, D, pos, in.rope_step, in.epsilon);
    } else {
        load16_f16(static_cast<const uint16_t*>(in.k) + src, xk);
        load16_f16(static_cast<const uint16_t*>(in.v) + src, xv);
    }
    int8_t qk[16], qv[16];
    float sk, sv;
    quantize16(xk, qk, sk);
    quantize16(xv, qv, sv);

    uint8_t* s_k = reinterpret_cast<uint8_t*>(s_tile);  // [32*D] K codes, slab order
    uint8_t* s_v = s_k + 32 * D;                         // [32][D] V codes, token-major
    uint16_t* s_s = reinterpret_cast<uint16_t*>(s_v + 32 * D);  // [2][32][D/32] scales
    const uint32_t d0 = q16 * 16;
    uint32_t packed[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        packed[w] = (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * w]))) |
                    (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * w + 1])) << 8) |
                    (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * w + 2])) << 16) |
                    (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * w + 3])) << 24);
    }
    *reinterpret_cast<uint2*>(s_k + k_code_offset(tl, d0, D)) = make_uint2(packed[0], packed[1]);
    *reinterpret_cast<uint2*>(s_k + k_code_offset(tl, d0 + 8, D)) = make_uint2(packed[2], packed[3]);
    // V codes row-major here (one 16-byte store, no bank conflicts); the slab's
    // token-interleaved order is gathered on the way out.
    uint32_t vpk[4];
#pragma unroll
    for (int w = 0; w < 4; ++w)
        vpk[w] = (static_cast<uint32_t>(static_cast<uint8_t>(qv[4 * w]))) |
                 (static_cast<uint32_t>(static_cast<uint8_t>(qv[4 * w + 1])) << 8) |
                 (static_cast<uint32_t>(static_cast<uint8_t>(qv[4 * w + 2])) << 16) |
                 (static_cast<uint32_t>(static_cast<uint8_t>(qv[4 * w + 3])) << 24);
    *reinterpret_cast<uint4*>(s_v + tl * D + d0) = make_uint4(vpk[0], vpk[1], vpk[2], vpk[3]);
    if ((q16 & 1) == 0) {
        s_s[tl * (D / 32) + d0 / 32] = f32_to_f16_bits(sk);
        s_s[32 * (D / 32) + tl * (D / 32) + d0 / 32] = f32_to_f16_bits(sv);
    }
    __syncthreads();

    const uint32_t pos0 = base_position + blockIdx.x * 32;
    const size_t slab = slab_of(g, seq, pos0, head);
    const uint32_t tp0 = pos0 % g.page_tokens;
    const size_t slab_bytes = static_cast<size_t>(g.page_tokens) * D;
    uint4* kdst = reinterpret_cast<uint4*>(g.k_codes + slab * slab_bytes + static_cast<size_t>(tp0) * D);
    uint4* vdst = reinterpret_cast<uint4*>(g.v_codes + slab * slab_bytes + static_cast<size_t>(tp0) * D);
    const uint32_t chunks = 32 * D / 16;  // 16-byte chunks per code region
    for (uint32_t c = threadIdx.x; c < chunks; c += blockDim.x) {
        kdst[c] = s_tile[c];
        // V chunk c: dim d = c/2, slab bytes 16*(c%2) .. +15 of that dim hold tokens
        // 16J + 4G + I at 8G + 4J + I, G = 2*(c%2) + {0, 1}: four 4-token runs.
        const uint32_t d = c / 2, g0 = 2 * (c % 2);
        uint32_t w[4];
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k) {
            const uint32_t t0 = 16 * (k % 2) + 4 * (g0 + k / 2);
            w[k] = static_cast<uint32_t>(s_v[t0 * D + d]) | (static_cast<uint32_t>(s_v[(t0 + 1) * D + d]) << 8) |
                   (static_cast<uint32_t>(s_v[(t0 + 2) * D + d]) << 16) |
                   (static_cast<uint32_t>(s_v[(t0 + 3) * D + d]) << 24);
        }
        vdst[c] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    const uint32_t schunks = 32 * (D / 32) * 2 / 16;  // 16-byte chunks per scale region
    const size_t sidx = (slab * g.page_tokens + tp0) * (D / 32);
    if (threadIdx.x < 2 * schunks) {
        const uint32_t kind = threadIdx.x / schunks, c = threadIdx.x % schunks;
        uint16_t* sdst = (kind == 0 ? g.k_scales : g.v_scales) + sidx;
        reinterpret_cast<uint4*>(sdst)[c] = s_tile[2 * chunks + kind * schunks + c];
    }
}

// Stop tokens of one decode-state advance (passed by value).
struct StopSet {
    uint32_t count;
    uint32_t token[8];
};

// After a decode step: record the step's token, raise `stop` on a stop token or
// the generation limit, and move to the next position
// (qwen35_decode_state_advance_kernel, gfx906/kernels/qwen3_primitives.hip:4417-4429).
__global__ void decode_state_advance_kernel(miikv_decode_state* st, uint32_t* token_output, uint32_t capacity,
                                            StopSet stops) {
    if (blockIdx.x != 0 || threadIdx.x != 0) return;
    const uint32_t generated = st->generated;
    const uint32_t tok = st->current_token;
    if (token_output != nullptr && generated < capacity) token_output[generated] = tok;
    bool stop = st->stop != 0 || generated + 1 >= st->max_generated;
    for (uint32_t i = 0; i < stops.count; ++i) stop = stop || tok == stops.token[i];
    st->stop = stop ? 1u : 0u;
    st->position += 1;
    st->generated = generated + 1;
}

// Tiled -> canonical (export) or canonical -> tiled (import), one thread per
// (token, kv_head, 16-dim group).
template <bool EXPORT>
__global__ void __launch_bounds__(256) canonical_kernel(
    Geo g, uint32_t seq, uint32_t t0, uint32_t count, int8_t* kc, uint16_t* ks, int8_t* vc,
    uint16_t* vs) {
    const uint32_t D = g.head_dim;
    const uint32_t groups = D / 16;
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(count) * g.kv_heads * groups;
    if (gid >= total) return;
    const uint32_t q16 = static_cast<uint32_t>(gid % groups);
    const uint64_t r = gid / groups;
    const uint32_t t = static_cast<uint32_t>(r % count);
    const uint32_t head = static_cast<uint32_t>(r / count);
    const uint32_t pos = t0 + t;
    const size_t slab = slab_of(g, seq, pos, head);
    const uint32_t tp = pos % g.page_tokens;
    const size_t slab_bytes = static_cast<size_t>(g.page_tokens) * D;
    const uint32_t d0 = q16 * 16;
    const size_t crow = (static_cast<size_t>(head) * count + t) * D + d0;
    int8_t* kslab = g.k_codes + slab * slab_bytes;
    int8_t* vslab = g.v_codes + slab * slab_bytes;
    const size_t sidx = (slab * g.page_tokens + tp) * (D / 32) + d0 / 32;
    const size_t csidx = (static_cast<size_t>(head) * count + t) * (D / 32) + d0 / 32;
    // fp16 planes: canonical rows are fp16 [kv_head][count][D]; no scales.
    uint16_t* kslab16 = reinterpret_cast<uint16_t*>(g.k_codes) + slab * slab_bytes;
    uint16_t* vslab16 = reinterpret_cast<uint16_t*>(g.v_codes) + slab * slab_bytes;
    uint16_t* kc16 = reinterpret_cast<uint16_t*>(kc);
    uint16_t* vc16 = reinterpret_cast<uint16_t*>(vc);
    if (g.k_f16) {
        if (kc != nullptr) {
            uint4* kslab4_lo = reinterpret_cast<uint4*>(kslab16 + k_code_offset(tp, d0, D));
            uint4* kslab4_hi = reinterpret_cast<uint4*>(kslab16 + k_code_offset(tp, d0 + 8, D));
            uint4* krow = reinterpret_cast<uint4*>(kc16 + crow);
            if (EXPORT) {
                krow[0] = *kslab4_lo;
                krow[1] = *kslab4_hi;
            } else {
                *kslab4_lo = krow[0];
                *kslab4_hi = krow[1];
            }
        }
        kc = nullptr;
        ks = nullptr;
    }
    if (g.v_f16) {
        if (vc != nullptr) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (EXPORT) vc16[crow + i] = vslab16[v_code_offset(tp, d0 + i, D)];
                else vslab16[v_code_offset(tp, d0 + i, D)] = vc16[crow + i];
            }
        }
        vc = nullptr;
        vs = nullptr;
    }
    if (EXPORT) {
        if (kc != nullptr) {
            const uint2 a = *reinterpret_cast<const uint2*>(kslab + k_code_offset(tp, d0, D));
            const uint2 b = *reinterpret_cast<const uint2*>(kslab + k_code_offset(tp, d0 + 8, D));
            *reinterpret_cast<uint4*>(kc + crow) = make_uint4(a.x, a.y, b.x, b.y);
        }
        if (vc != nullptr) {
            uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 16; ++i)
                w[i / 4] |= static_cast<uint32_t>(static_cast<uint8_t>(vslab[v_code_offset(tp, d0 + i, D)]))
                            << (8 * (i % 4));
            *reinterpret_cast<uint4*>(vc + crow) = make_uint4(w[0], w[1], w[2], w[3]);
        }
        if ((q16 & 1) == 0) {
            if (ks != nullptr) ks[csidx] = g.k_scales[sidx];
            if (vs != nullptr) vs[csidx] = g.v_scales[sidx];
        }
    } else {
        if (kc != nullptr) {
            const uint4 a = *reinterpret_cast<const uint4*>(kc + crow);
            *reinterpret_cast<uint2*>(kslab + k_code_offset(tp, d0, D)) = make_uint2(a.x, a.y);
            *reinterpret_cast<uint2*>(kslab + k_code_offset(tp, d0 + 8, D)) = make_uint2(a.z, a.w);
        }
        if (vc != nullptr) {
            const uint4 a = *reinterpret_cast<const uint4*>(vc + crow);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int i = 0; i < 16; ++i)
                vslab[v_code_offset(tp, d0 + i, D)] = static_cast<int8_t>((w[i / 4] >> (8 * (i % 4))) & 0xffu);
        }
        if ((q16 & 1) == 0) {
            if (ks != nullptr) g.k_scales[sidx] = ks[csidx];
            if (vs != nullptr) g.v_scales[sidx] = vs[csidx];
        }
    }
}

// Tiled -> dequantised fp32 rows [kv_head][count][head_dim], value = float(code) *
// float(scale) (src/prefill_v2/kv_cache.cpp:161-169), one thread per (token, kv head,
// 16-dim group).
__global__ void __launch_bounds__(256) dequant_kernel(Geo g, uint32_t seq, uint32_t t0, uint32_t count,
                                                      float* kout, float* vout) {
    const uint32_t D = g.head_dim;
    const uint32_t groups = D / 16;
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t total = static_cast<uint64_t>(count) * g.kv_heads * groups;
    if (gid >= total) return;
    const uint32_t q16 = static_cast<uint32_t>(gid % groups);
    const uint64_t r = gid / groups;
    const uint32_t t = static_cast<uint32_t>(r % count);
    const uint32_t head = static_cast<uint32_t>(r / count);
    const uint32_t pos = t0 + t;
    const size_t slab = slab_of(g, seq, pos, head);
    const uint32_t tp = pos % g.page_tokens;
    const size_t slab_bytes = static_cast<size_t>(g.page_tokens) * D;
    const uint32_t d0 = q16 * 16;
    const size_t row = (static_cast<size_t>(head) * count + t) * D + d0;
    const size_t sidx = (slab * g.page_tokens + tp) * (D / 32) + d0 / 32;
    if (kout != nullptr && g.k_f16) {
        const uint16_t* kslab = reinterpret_cast<const uint16_t*>(g.k_codes) + slab * slab_bytes;
        float x[16];
        unpack16_f16({*reinterpret_cast<const uint4*>(kslab + k_code_offset(tp, d0, D)),
                      *reinterpret_cast<const uint4*>(kslab + k_code_offset(tp, d0 + 8, D))}, x);
        float4* o = reinterpret_cast<float4*>(kout + row);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
        kout = nullptr;
    }
    if (vout != nullptr && g.v_f16) {
        const uint16_t* vslab = reinterpret_cast<const uint16_t*>(g.v_codes) + slab * slab_bytes;
        float4* o = reinterpret_cast<float4*>(vout + row);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o[i] = make_float4(f16_bits_to_f32(vslab[v_code_offset(tp, d0 + 4 * i, D)]),
                               f16_bits_to_f32(vslab[v_code_offset(tp, d0 + 4 * i + 1, D)]),
                               f16_bits_to_f32(vslab[v_code_offset(tp, d0 + 4 * i + 2, D)]),
                               f16_bits_to_f32(vslab[v_code_offset(tp, d0 + 4 * i + 3, D)]));
        vout = nullptr;
    }
    if (kout != nullptr) {
        const int8_t* kslab = g.k_codes + slab * slab_bytes;
        const uint2 a = *reinterpret_cast<const uint2*>(kslab + k_code_offset(tp, d0, D));
        const uint2 b = *reinterpret_cast<const uint2*>(kslab + k_code_offset(tp, d0 + 8, D));
        const uint32_t w[4] = {a.x, a.y, b.x, b.y};
        const float sc = f16_bits_to_f32(g.k_scales[sidx]);
        float4* o = reinterpret_cast<float4*>(kout + row);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o[i] = make_float4(static_cast<float>(static_cast<int8_t>(w[i] & 0xffu)) * sc,
                               static_cast<float>(static_cast<int8_t>((w[i] >> 8) & 0xffu)) * sc,
                               static_cast<float>(static_cast<int8_t>((w[i] >> 16) & 0xffu)) * sc,
                               static_cast<float>(static_cast<int8_t>(w[i] >> 24)) * sc);
    }
    if (vout != nullptr) {
        const int8_t* vslab = g.v_codes + slab * slab_bytes;
        const float sc = f16_bits_to_f32(g.v_scales[sidx]);
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = static_cast<float>(vslab[v_code_offset(tp, d0 + i, D)]) * sc;
        float4* o = reinterpret_cast<float4*>(vout + row);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
    }
}

// Copy [src, src+bytes) to dst with 16-byte vectors; `bytes` is a multiple of 16.
__device__ __forceinline__ void copy16(uint4* __restrict__ dst, const uint4* __restrict__ src, uint64_t n16,
                                       uint64_t start, uint64_t stride) {
    for (uint64_t i = start; i < n16; i += stride) dst[i] = src[i];
}

// grid (blocks, n_pages): block y copies page src_pages[y] -> dst_pages[y], all four planes.
__global__ void __launch_bounds__(256) copy_pages_kernel(Geo g, const int32_t* __restrict__ srcp,
                                                         const int32_t* __restrict__ dstp) {
    const uint32_t i = blockIdx.y;
    const size_t s = static_cast<size_t>(srcp[i]);
    const size_t d = static_cast<size_t>(dstp[i]);
    const uint64_t code_bytes = static_cast<uint64_t>(g.kv_heads) * g.page_tokens * g.head_dim;
    const uint64_t kbytes = code_bytes * (g.k_f16 ? 2 : 1), vbytes = code_bytes * (g.v_f16 ? 2 : 1);
    const uint64_t scale_bytes = static_cast<uint64_t>(g.kv_heads) * g.page_tokens * (g.head_dim / 32) * 2;
    const uint64_t start = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    copy16(reinterpret_cast<uint4*>(g.k_codes + d * kbytes),
           reinterpret_cast<const uint4*>(g.k_codes + s * kbytes), kbytes / 16, start, stride);
    copy16(reinterpret_cast<uint4*>(g.v_codes + d * vbytes),
           reinterpret_cast<const uint4*>(g.v_codes + s * vbytes), vbytes / 16, start, stride);
    if (!g.k_f16)
        copy16(reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(g.k_scales) + d * scale_bytes),
               reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(g.k_scales) + s * scale_bytes),
               scale_bytes / 16, start, stride);
    if (!g.v_f16)
        copy16(reinterpret_cast<uint4*>(reinterpret_cast<uint8_t*>(g.v_scales) + d * scale_bytes),
               reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(g.v_scales) + s * scale_bytes),
               scale_bytes / 16, start, stride);
}

// grid (blocks, n): block y copies segment y.  16-byte path when both ends and
// the size are 16-byte aligned, byte path otherwise.
__global__ void __launch_bounds__(256) copy_segments_kernel(const miikv_segment* __restrict__ segs) {
    const miikv_segment sg = segs[blockIdx.y];
    const uint64_t start = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    const bool aligned = ((reinterpret_cast<uintptr_t>(sg.dst) | reinterpret_cast<uintptr_t>(sg.src) | sg.bytes) & 15u) == 0;
    if (aligned) {
        copy16(reinterpret_cast<uint4*>(sg.dst), reinterpret_cast<const uint4*>(sg.src), sg.bytes / 16, start, stride);
    } else {
        uint8_t* d = reinterpret_cast<uint8_t*>(sg.dst);
        const uint8_t* s = reinterpret_cast<const uint8_t*>(sg.src);
        for (uint64_t i = start; i < sg.bytes; i += stride) d[i] = s[i];
    }
}

// Each thread reads one 16-byte vector of the source once and writes it to
// every destination, so the source is fetched from HBM once per clone batch.
__global__ void __launch_bounds__(256) clone_state_kernel(void* const* __restrict__ dsts,
                                                          const uint4* __restrict__ src, uint64_t n16,
                                                          uint32_t n) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const uint4 x = src[i];
        for (uint32_t k = 0; k < n; ++k) reinterpret_cast<uint4*>(dsts[k])[i] = x;
    }
}

// Read-only streaming probe: each workgroup reads a contiguous span with 16-byte
// nontemporal loads (8 in flight per thread) and folds it into one word.
__global__ void __launch_bounds__(256) stream_read_kernel(const uint4* __restrict__ src, uint64_t per_block,
                                                          uint32_t* __restrict__ sink) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v* base = reinterpret_cast<const u4v*>(src) + blockIdx.x * per_block;
    uint32_t acc = 0;
    for (uint64_t i = threadIdx.x; i < per_block; i += 256 * 8) {
        u4v v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint64_t j = i + static_cast<uint64_t>(u) * 256;
            v[u] = j < per_block ? __builtin_nontemporal_load(base + j) : u4v{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    acc ^= __shfl_xor(acc, 1, 64);
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

int launch_status() { return hip_status(hipGetLastError()); }

}  // namespace
}  // namespace miikv

using namespace miikv;

extern "C" uint32_t miikv_abi_version(void) { return MIIKV_ABI_VERSION; }

extern "C" const char* miikv_status_string(miikv_status s) {
    switch (s) {
        case MIIKV_OK: return "ok";
        case MIIKV_EINVAL: return "invalid argument";
        case MIIKV_EUNSUPPORTED: return "unsupported configuration";
        case MIIKV_EWORKSPACE: return "workspace missing or too small";
        default: return s < 0 ? hipGetErrorString(static_cast<hipError_t>(-s)) : "unknown status";
    }
}

extern "C" miikv_status miikv_plane_bytes(const miikv_view* view, uint64_t* code_bytes, uint64_t* scale_bytes) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    const uint64_t tokens = static_cast<uint64_t>(view->num_pages) * view->page_tokens * view->kv_heads;
    if (code_bytes) *code_bytes = tokens * view->head_dim;
    if (scale_bytes) *scale_bytes = tokens * (view->head_dim / 32) * 2;
    return MIIKV_OK;
}

// Token count from which a host-positioned append sends its whole 32-token groups to
// append_tile_kernel (the partial groups at either end go through append_kernel).
constexpr uint32_t kTileAppendMin = 64;

template <bool F32>
static AppendIn advance_rows(AppendIn in, uint64_t tokens, uint32_t kv_heads, uint32_t D) {
    const uint64_t elems = tokens * kv_heads * D;
    const size_t esize = F32 ? sizeof(float) : sizeof(uint16_t);
    in.k = static_cast<const char*>(in.k) + elems * esize;
    in.v = static_cast<const char*>(in.v) + elems * esize;
    return in;
}

template <bool F32>
static miikv_status launch_rows(const miikv_view* view, const AppendIn& in, uint32_t rows_tokens, uint32_t base,
                                uint32_t seq, const miikv_prefill_state* ps, const miikv_decode_state* ds,
                                const uint32_t* positions, void* stream) {
    const uint64_t threads = static_cast<uint64_t>(rows_tokens) * view->kv_heads * (view->head_dim / 16);
    if (threads == 0) return MIIKV_OK;
    const uint64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffu) return MIIKV_EINVAL;
    hipLaunchKernelGGL(append_kernel<F32>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), make_geo(*view), in, rows_tokens, base, seq, ps, ds,
                       positions);
    return launch_status();
}

template <bool F32>
static miikv_status launch_append(const miikv_view* view, const AppendIn& in, uint32_t rows_tokens, uint32_t base,
                                  uint32_t seq, const miikv_prefill_state* ps, const miikv_decode_state* ds,
                                  const uint32_t* positions, void* stream) {
    // Positions known on the host: [head partial group][whole groups][tail partial group].
    // (The grouped store assembles q8 codes and scales; caches with an fp16 plane take
    // the per-row kernel.)
    if (ps == nullptr && ds == nullptr && positions == nullptr && rows_tokens >= kTileAppendMin &&
        view->quant_mode == MIIKV_KV_Q8_Q8) {
        const uint32_t D = view->head_dim;
        const uint32_t head = (32 - base % 32) % 32;
        const uint32_t whole = (rows_tokens - head) / 32;
        const uint32_t tail = rows_tokens - head - whole * 32;
        int st = launch_rows<F32>(view, in, head, base, seq, nullptr, nullptr, nullptr, stream);
        if (st != MIIKV_OK) return st;
        if (whole > 0) {
            const size_t lds = 2 * 32 * D + 2 * 32 * (D / 32) * sizeof(uint16_t);
            hipLaunchKernelGGL(append_tile_kernel<F32>, dim3(whole, view->kv_heads), dim3(32 * (D / 16)), lds,
                               static_cast<hipStream_t>(stream), make_geo(*view),
                               advance_rows<F32>(in, head, view->kv_heads, D), base + head, seq);
            st = launch_status();
            if (st != MIIKV_OK) return st;
        }
        return launch_rows<F32>(view, advance_rows<F32>(in, head + 32ull * whole, view->kv_heads, D), tail,
                                base + head + whole * 32, seq, nullptr, nullptr, nullptr, stream);
    }
    return launch_rows<F32>(view, in, rows_tokens, base, seq, ps, ds, positions, stream);
}

static AppendIn f16_rows(const uint16_t* k, const uint16_t* v) {
    AppendIn in{};
    in.k = k;
    in.v = v;
    return in;
}

extern "C" miikv_status miikv_append_f16(const miikv_view* view, const uint16_t* k, const uint16_t* v,
                                         uint32_t token_count, uint32_t base_position, uint32_t seq,
                                         const miikv_prefill_state* prefill_state,
                                         const miikv_decode_state* decode_state, void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (k == nullptr || v == nullptr) return MIIKV_EINVAL;
    if (decode_state != nullptr && prefill_state == nullptr) token_count = 1;
    if (prefill_state == nullptr && decode_state == nullptr &&
        static_cast<uint64_t>(base_position) + token_count > view_seq_capacity(view))
        return MIIKV_EINVAL;
    if (view->layout == MIIKV_LAYOUT_CONTIGUOUS && seq != 0) return MIIKV_EINVAL;
    return launch_append<false>(view, f16_rows(k, v), token_count, base_position, seq, prefill_state, decode_state,
                                nullptr, stream);
}

extern "C" miikv_status miikv_append_f32(const miikv_view* view, const float* k, const float* v,
                                         const float* k_norm_weight, uint32_t token_count, uint32_t base_position,
                                         uint32_t seq, float theta, float epsilon,
                                         const miikv_prefill_state* prefill_state,
                                         const miikv_decode_state* decode_state, void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (k == nullptr || v == nullptr) return MIIKV_EINVAL;
    if (k_norm_weight != nullptr && (view->head_dim < 64 || !std::isfinite(theta) || !std::isfinite(epsilon)))
        return MIIKV_EINVAL;
    if (decode_state != nullptr && prefill_state == nullptr) token_count = 1;
    if (prefill_state == nullptr && decode_state == nullptr &&
        static_cast<uint64_t>(base_position) + token_count > view_seq_capacity(view))
        return MIIKV_EINVAL;
    if (view->layout == MIIKV_LAYOUT_CONTIGUOUS && seq != 0) return MIIKV_EINVAL;
    AppendIn in{};
    in.k = k;
    in.v = v;
    in.k_norm_weight = k_norm_weight;
    in.rope_step = powf(theta, -2.0f / 64.0f);
    in.epsilon = epsilon;
    return launch_append<true>(view, in, token_count, base_position, seq, prefill_state, decode_state, nullptr,
                               stream);
}

extern "C" miikv_status miikv_append_batch_f16(const miikv_view* view, const uint16_t* k, const uint16_t* v,
                                               uint32_t batch, const uint32_t* d_positions, void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (k == nullptr || v == nullptr || d_positions == nullptr) return MIIKV_EINVAL;
    if (view->layout == MIIKV_LAYOUT_CONTIGUOUS && batch > 1) return MIIKV_EINVAL;
    return launch_append<false>(view, f16_rows(k, v), batch, 0, 0, nullptr, nullptr, d_positions, stream);
}

template <bool EXPORT>
static miikv_status launch_canonical(const miikv_view* view, uint32_t seq, uint32_t t0, uint32_t count, int8_t* kc,
                                     uint16_t* ks, int8_t* vc, uint16_t* vs, void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (static_cast<uint64_t>(t0) + count > view_seq_capacity(view)) return MIIKV_EINVAL;
    if (view->layout == MIIKV_LAYOUT_CONTIGUOUS && seq != 0) return MIIKV_EINVAL;
    const uint64_t threads = static_cast<uint64_t>(count) * view->kv_heads * (view->head_dim / 16);
    if (threads == 0) return MIIKV_OK;
    const uint64_t blocks = (threads + 255) / 256;
    hipLaunchKernelGGL(canonical_kernel<EXPORT>, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), make_geo(*view), seq, t0, count, kc, ks, vc, vs);
    return launch_status();
}

extern "C" miikv_status miikv_export_canonical(const miikv_view* view, uint32_t seq, uint32_t t0, uint32_t count,
                                               int8_t* k_codes, uint16_t* k_scales, int8_t* v_codes,
                                               uint16_t* v_scales, void* stream) {
    return launch_canonical<true>(view, seq, t0, count, k_codes, k_scales, v_codes, v_scales, stream);
}

extern "C" miikv_status miikv_import_canonical(const miikv_view* view, uint32_t seq, uint32_t t0, uint32_t count,
                                               const int8_t* k_codes, const uint16_t* k_scales,
                                               const int8_t* v_codes, const uint16_t* v_scales, void* stream) {
    return launch_canonical<false>(view, seq, t0, count, const_cast<int8_t*>(k_codes),
                                   const_cast<uint16_t*>(k_scales), const_cast<int8_t*>(v_codes),
                                   const_cast<uint16_t*>(v_scales), stream);
}

extern "C" miikv_status miikv_export_dequant(const miikv_view* view, uint32_t seq, uint32_t t0, uint32_t count,
                                             float* k_out, float* v_out, void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (static_cast<uint64_t>(t0) + count > view_seq_capacity(view)) return MIIKV_EINVAL;
    if (view->layout == MIIKV_LAYOUT_CONTIGUOUS && seq != 0) return MIIKV_EINVAL;
    if ((reinterpret_cast<uintptr_t>(k_out) | reinterpret_cast<uintptr_t>(v_out)) & 15u) return MIIKV_EINVAL;
    const uint64_t threads = static_cast<uint64_t>(count) * view->kv_heads * (view->head_dim / 16);
    if (threads == 0 || (k_out == nullptr && v_out == nullptr)) return MIIKV_OK;
    const uint64_t blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffu) return MIIKV_EINVAL;
    hipLaunchKernelGGL(dequant_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), make_geo(*view), seq, t0, count, k_out, v_out);
    return launch_status();
}

extern "C" miikv_status miikv_copy_pages(const miikv_view* view, const int32_t* d_src_pages,
                                         const int32_t* d_dst_pages, uint32_t n, void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (n == 0) return MIIKV_OK;
    if (d_src_pages == nullptr || d_dst_pages == nullptr || n > 65535u) return MIIKV_EINVAL;
    const uint64_t code16 = static_cast<uint64_t>(view->kv_heads) * view->page_tokens * view->head_dim / 16;
    uint32_t blocks = static_cast<uint32_t>((code16 + 255) / 256);
    if (blocks > 64) blocks = 64;
    hipLaunchKernelGGL(copy_pages_kernel, dim3(blocks, n), dim3(256), 0, static_cast<hipStream_t>(stream),
                       make_geo(*view), d_src_pages, d_dst_pages);
    return launch_status();
}

extern "C" miikv_status miikv_copy_segments(const miikv_segment* d_segments, uint32_t n, void* stream) {
    if (n == 0) return MIIKV_OK;
    if (d_segments == nullptr || n > 65535u) return MIIKV_EINVAL;
    hipLaunchKernelGGL(copy_segments_kernel, dim3(128, n), dim3(256), 0, static_cast<hipStream_t>(stream),
                       d_segments);
    return launch_status();
}

extern "C" miikv_status miikv_clone_state(void* const* d_dsts, const void* src, uint64_t bytes, uint32_t n,
                                          void* stream) {
    if (n == 0 || bytes == 0) return MIIKV_OK;
    if (d_dsts == nullptr || src == nullptr || (bytes & 15u) != 0 || (reinterpret_cast<uintptr_t>(src) & 15u) != 0)
        return MIIKV_EINVAL;
    const uint64_t n16 = bytes / 16;
    uint64_t blocks = (n16 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(clone_state_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), d_dsts, reinterpret_cast<const uint4*>(src), n16, n);
    return launch_status();
}

extern "C" miikv_status miikv_stream_read(const void* src, uint64_t bytes, uint32_t* sink, uint32_t blocks,
                                          void* stream) {
    if (src == nullptr || sink == nullptr || blocks == 0 || (bytes % (16ull * blocks)) != 0 ||
        (reinterpret_cast<uintptr_t>(src) & 15u) != 0)
        return MIIKV_EINVAL;
    hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<const uint4*>(src), bytes / 16 / blocks, sink);
    return launch_status();
}

extern "C" miikv_status miikv_decode_state_advance(miikv_decode_state* state, uint32_t* token_output,
                                                   uint32_t capacity, const uint32_t* stop_tokens,
                                                   uint32_t stop_count, void* stream) {
    if (state == nullptr || stop_count > 8 || (stop_count > 0 && stop_tokens == nullptr)) return MIIKV_EINVAL;
    StopSet stops{};
    stops.count = stop_count;
    for (uint32_t i = 0; i < stop_count; ++i) stops.token[i] = stop_tokens[i];
    hipLaunchKernelGGL(decode_state_advance_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), state,
                       token_output, capacity, stops);
    return launch_status();
}
