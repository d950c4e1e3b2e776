// Split-K GQA decode attention over the tiled q8_0 cache (gfx950, wave64, MFMA).
//
// Work decomposition.  A workgroup of 4 waves owns one (sequence, kv head,
// split); a split is 4 * chunks_per_wave chunks of 64 tokens and each wave
// streams `chunks_per_wave` consecutive chunks.  All G = q_heads / kv_heads
// query heads of the kv head are served by the same wave, so every K/V byte
// is read from HBM exactly once.
//
// Per 64-token chunk a wave computes, for 4 tiles of 16 tokens:
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
// wide kernel merges the splits.  Two launches on one stream need no
// cross-workgroup synchronisation: a grid-wide arrival counter would need an
// agent-scope release (an L2 write-back on every XCD) per workgroup, which
// measured slower than the second launch.  The merge follows the reference
// combine (gfx906/kernels/qwen3_primitives.hip:2295-2385): g = max m_s,
// L = sum l_s e^{m_s-g}, out = sum acc_s e^{m_s-g} / L, 0 when L == 0,
// gated = out * sigmoid(gate).
#include "miikv_common.hpp"

#include <cmath>

namespace miikv {

int validate_view(const miikv_view* v);
uint64_t view_seq_capacity(const miikv_view* v);

namespace {

constexpr uint32_t kWavesPerWg = 4;
constexpr uint32_t kTargetWaves = 256 * 8;  // 256 CUs x 8 resident waves
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeArgs {
    Geo g;
    const void* q;
    uint32_t q_heads;
    uint32_t group;  // query heads per kv head (<= 16)
    float scale_log2;
    const uint32_t* len_ptr;
    uint32_t len_stride;
    uint32_t len_add;
    uint32_t max_context;
    uint32_t cpw;         // chunks per wave
    uint32_t max_splits;  // == gridDim.x
    float* part;          // [batch][kv_heads][max_splits][group*(D+2)]
    float* out;
    const float* gate;
    float* gated_out;
};

__device__ __forceinline__ float wave_max_xor_16_32(float x) {
    x = fmaxf(x, __shfl_xor(x, 16, 64));
    x = fmaxf(x, __shfl_xor(x, 32, 64));
    return x;
}

__device__ __forceinline__ float exp2_safe(float x) { return exp2f(x); }  // exp2(-inf) == 0

// Floats in one split's partial record: O [G*D], m [G], l [G], padded to 4.
__host__ __device__ __forceinline__ uint32_t record_floats(uint32_t G, uint32_t D) {
    return G * D + ((2 * G + 3) / 4) * 4;
}

template <uint32_t D, bool QF32>
__global__ void __launch_bounds__(256) decode_kernel(DecodeArgs a) {
    constexpr uint32_t NB = D / 32;   // q8_0 blocks per row
    constexpr uint32_t NC = D / 64;   // 16-byte K loads per tile row group
    constexpr uint32_t NM = D / 16;   // V M-tiles (16 dims each)
    extern __shared__ float smem[];

    const uint32_t split = blockIdx.x;
    const uint32_t h = blockIdx.y;
    const uint32_t b = blockIdx.z;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63;
    const uint32_t g4 = lane >> 4;
    const uint32_t n = lane & 15;
    const uint32_t G = a.group;
    const Geo& geo = a.g;

    uint32_t L = a.len_ptr[static_cast<size_t>(b) * a.len_stride] + a.len_add;
    if (L > a.max_context) L = a.max_context;
    const uint32_t tps = kWavesPerWg * a.cpw * kChunk;
    const uint32_t nsplit = (L + tps - 1) / tps;
    if (split >= nsplit) return;  // includes L == 0 (the combine kernel writes zeros)

    // ---- Q fragments (B operand of the QK MFMA): lane (g4, n) holds head n,
    // dims 32*blk + 8*g4 .. +7 of every block.
    half8 qf[NB];
    half8 ql[QF32 ? NB : 1];
    {
        const size_t qrow = (static_cast<size_t>(b) * a.q_heads + static_cast<size_t>(h) * G + n) * D;
#pragma unroll
        for (uint32_t blk = 0; blk < NB; ++blk) {
            half8 v = {};
            half8 lo = {};
            if (n < G) {
                if (QF32) {
                    const float* qp = static_cast<const float*>(a.q) + qrow + blk * 32 + g4 * 8;
                    const float4 x0 = *reinterpret_cast<const float4*>(qp);
                    const float4 x1 = *reinterpret_cast<const float4*>(qp + 4);
                    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const _Float16 hi = static_cast<_Float16>(xs[i]);
                        v[i] = hi;
                        lo[i] = static_cast<_Float16>(xs[i] - static_cast<float>(hi));
                    }
                } else {
                    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qrow + blk * 32 + g4 * 8;
                    v = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(qp));
                }
            }
            qf[blk] = v;
            if (QF32) ql[QF32 ? blk : 0] = lo;
        }
    }

    float m_run = -INFINITY;
    float l_run = 0.0f;
    float4v O[NM];
#pragma unroll
    for (uint32_t mt = 0; mt < NM; ++mt) O[mt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    const uint32_t nchunks = (L + kChunk - 1) / kChunk;
    const uint32_t c_begin = (split * kWavesPerWg + wave) * a.cpw;
#ifdef MIIKV_EXP_NO_LOOP
    const uint32_t c_end = c_begin;
#else
    const uint32_t c_end = min(c_begin + a.cpw, nchunks);
#endif
    const size_t slab_bytes = static_cast<size_t>(geo.page_tokens) * D;

    for (uint32_t c = c_begin; c < c_end; ++c) {
        const uint32_t tok0 = c * kChunk;
        const size_t slab = slab_of(geo, b, tok0, h);
        const uint32_t tp0 = tok0 % geo.page_tokens;
        const int8_t* kb = geo.k_codes + slab * slab_bytes + static_cast<size_t>(tp0) * D;
        const int8_t* vb = geo.v_codes + slab * slab_bytes + static_cast<size_t>(tp0) * D;
        const uint16_t* ksb = geo.k_scales + (slab * geo.page_tokens + tp0) * NB;
        const uint16_t* vsb = geo.v_scales + (slab * geo.page_tokens + tp0) * NB;

        // Issue all loads of the chunk up front.
        uint4 kw[4][NC];
#pragma unroll
        for (uint32_t J = 0; J < 4; ++J)
#pragma unroll
            for (uint32_t cc = 0; cc < NC; ++cc)
                kw[J][cc] = *reinterpret_cast<const uint4*>(kb + J * 16 * D + cc * 1024 + g4 * 256 + n * 16);
        uint4 vw[NM];
#pragma unroll
        for (uint32_t mt = 0; mt < NM; ++mt)
            vw[mt] = *reinterpret_cast<const uint4*>(vb + (16 * mt + n) * 64 + g4 * 16);
        // Scales of tokens 16J + 4*g4 + i (i < 4), all blocks: 4*NB halves.
        uint4 ksw[4][NB / 2];
        uint4 vsw[4][NB / 2];
#pragma unroll
        for (uint32_t J = 0; J < 4; ++J)
#pragma unroll
            for (uint32_t w = 0; w < NB / 2; ++w) {
                ksw[J][w] = *reinterpret_cast<const uint4*>(ksb + (16 * J + 4 * g4) * NB + w * 8);
                vsw[J][w] = *reinterpret_cast<const uint4*>(vsb + (16 * J + 4 * g4) * NB + w * 8);
            }

        // ---- scores
        float s[4][4];
#pragma unroll
        for (uint32_t J = 0; J < 4; ++J) {
            const uint16_t* ks16 = reinterpret_cast<const uint16_t*>(&ksw[J][0]);
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t cc = 0; cc < NC; ++cc) {
                const uint4 w = kw[J][cc];
                const half8 a0 = codes8_to_half8(w.x, w.y);  // block 2cc
                const half8 a1 = codes8_to_half8(w.z, w.w);  // block 2cc+1
                float4v c0 = mfma_16x16x32(a0, qf[2 * cc], float4v{0.0f, 0.0f, 0.0f, 0.0f});
                float4v c1 = mfma_16x16x32(a1, qf[2 * cc + 1], float4v{0.0f, 0.0f, 0.0f, 0.0f});
                if (QF32) {
                    c0 = mfma_16x16x32(a0, ql[QF32 ? 2 * cc : 0], c0);
                    c1 = mfma_16x16x32(a1, ql[QF32 ? 2 * cc + 1 : 0], c1);
                }
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    acc[i] = fmaf(c0[i], f16_bits_to_f32(ks16[i * NB + 2 * cc]), acc[i]);
                    acc[i] = fmaf(c1[i], f16_bits_to_f32(ks16[i * NB + 2 * cc + 1]), acc[i]);
                }
            }
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                const bool valid = tok0 + 16 * J + 4 * g4 + i < L;
                s[J][i] = valid ? acc[i] * a.scale_log2 : -INFINITY;
            }
        }

        // ---- online softmax (per head n; the 4 lane groups share m)
        float cmax = s[0][0];
#pragma unroll
        for (uint32_t J = 0; J < 4; ++J)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) cmax = fmaxf(cmax, s[J][i]);
        cmax = wave_max_xor_16_32(cmax);
        const float m_new = fmaxf(m_run, cmax);
        const float alpha = exp2_safe(m_run - m_new);
        m_run = m_new;
        float psum = 0.0f;
#pragma unroll
        for (uint32_t J = 0; J < 4; ++J)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                s[J][i] = exp2_safe(s[J][i] - m_new);
                psum += s[J][i];
            }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (uint32_t mt = 0; mt < NM; ++mt) O[mt] *= alpha;

        // ---- O^T += V^T * (P^T scaled per block)
#pragma unroll
        for (uint32_t J = 0; J < 4; ++J) {
            const uint16_t* vs16 = reinterpret_cast<const uint16_t*>(&vsw[J][0]);
#pragma unroll
            for (uint32_t blk = 0; blk < NB; ++blk) {
                half4 pb;
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) {
                    const bool valid = tok0 + 16 * J + 4 * g4 + i < L;
                    const float w = s[J][i] * f16_bits_to_f32(vs16[i * NB + blk]);
                    pb[i] = static_cast<_Float16>(valid ? w : 0.0f);
                }
#pragma unroll
                for (uint32_t sub = 0; sub < 2; ++sub) {
                    const uint32_t mt = 2 * blk + sub;
                    const uint32_t word = (J == 0) ? vw[mt].x : (J == 1) ? vw[mt].y : (J == 2) ? vw[mt].z : vw[mt].w;
                    O[mt] = mfma_16x16x16(codes4_to_half4(word), pb, O[mt]);
                }
            }
        }
    }

    // ---- wave-level sums, then cross-wave combine in LDS.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    float* s_m = smem;                          // [4][16]
    float* s_l = smem + 64;                     // [4][16]
    float* s_O = smem + 128;                    // [4][G][D]
    __shared__ float s_M[16];
    if (g4 == 0) {
        s_m[wave * 16 + n] = m_run;
        s_l[wave * 16 + n] = l_run;
    }
    if (n < G) {
#pragma unroll
        for (uint32_t mt = 0; mt < NM; ++mt)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) s_O[(wave * G + n) * D + 16 * mt + 4 * g4 + i] = O[mt][i];
    }
    __syncthreads();

    // Partial record of one split: [O: G*D][m: G][l: G] padded to a multiple of 4 floats,
    // so every record starts 16-byte aligned.
    const uint32_t rec = record_floats(G, D);
    float* part = a.part + ((static_cast<size_t>(b) * geo.kv_heads + h) * a.max_splits) * rec;
    float* mine = part + static_cast<size_t>(split) * rec;
    if (tid < G) {
        float M = -INFINITY;
        for (uint32_t w = 0; w < kWavesPerWg; ++w) M = fmaxf(M, s_m[w * 16 + tid]);
        float Ls = 0.0f;
        for (uint32_t w = 0; w < kWavesPerWg; ++w) {
            const float mw = s_m[w * 16 + tid];
            if (mw != -INFINITY) Ls += s_l[w * 16 + tid] * exp2_safe(mw - M);
        }
        s_M[tid] = M;
        mine[G * D + tid] = M;
        mine[G * D + G + tid] = Ls;
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < G * D; idx += blockDim.x) {
        const uint32_t hn = idx / D;
        float o = 0.0f;
        for (uint32_t w = 0; w < kWavesPerWg; ++w) {
            const float mw = s_m[w * 16 + hn];
            if (mw != -INFINITY) o += s_O[w * G * D + idx] * exp2_safe(mw - s_M[hn]);
        }
        mine[idx] = o;
    }

    // ---- publish, and let the last workgroup of this (sequence, kv head) finish.
}



// Cross-split combine.  Workgroup (sequence * kv_heads + head, element block of 64)
// reads the partial records of every split of that (sequence, kv head): thread
// (e4 = tid & 15, sg = tid >> 4) folds splits sg, sg+16, ... for 4 consecutive
// elements with its own running max, so its loads are independent; the 16 split
// groups are merged in a fixed order through LDS (deterministic result).
template <uint32_t D>
__global__ void __launch_bounds__(256) combine_kernel(DecodeArgs a) {
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

    uint32_t L = a.len_ptr[static_cast<size_t>(b) * a.len_stride] + a.len_add;
    if (L > a.max_context) L = a.max_context;
    const uint32_t tps = kWavesPerWg * a.cpw * kChunk;
    const uint32_t nsplit = (L + tps - 1) / tps;
    const uint32_t rec = record_floats(G, D);
    const float* part = a.part + (static_cast<size_t>(bh) * a.max_splits) * rec;

    float mloc = -INFINITY;
    float lsum = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
    for (uint32_t sp = sg; sp < nsplit; sp += 16) {
        const float* r = part + static_cast<size_t>(sp) * rec;
        const float ms = r[GD + hn];
        const float ls = r[GD + G + hn];
        const float4 v = active ? *reinterpret_cast<const float4*>(r + e) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float mn = fmaxf(mloc, ms);
        const float fo = exp2_safe(mloc - mn);  // 0 on the first split
        const float fs = exp2_safe(ms - mn);
        mloc = mn;
        lsum = lsum * fo + ls * fs;
        acc.x = acc.x * fo + v.x * fs;
        acc.y = acc.y * fo + v.y * fs;
        acc.z = acc.z * fo + v.z * fs;
        acc.w = acc.w * fo + v.w * fs;
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
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        const size_t oi = out_row0 + e + k;
        if (a.out) a.out[oi] = vals[k];
        if (a.gate && a.gated_out) a.gated_out[oi] = vals[k] * (1.0f / (1.0f + expf(-a.gate[oi])));
    }
}

struct Plan {
    uint32_t cpw;
    uint32_t splits;
    uint64_t counter_bytes;
    uint64_t part_bytes;
};

Plan make_plan(const miikv_view* v, uint32_t q_heads, uint32_t batch, uint32_t max_context) {
    Plan p;
    const uint64_t chunks = (static_cast<uint64_t>(max_context) + kChunk - 1) / kChunk;
    const uint64_t waves = chunks * v->kv_heads * batch;
    uint64_t cpw = (waves + kTargetWaves - 1) / kTargetWaves;
    if (cpw < 1) cpw = 1;
    if (cpw > 64) cpw = 64;
    p.cpw = static_cast<uint32_t>(cpw);
    const uint64_t tps = kWavesPerWg * cpw * kChunk;
    p.splits = static_cast<uint32_t>((static_cast<uint64_t>(max_context) + tps - 1) / tps);
    if (p.splits == 0) p.splits = 1;
    const uint64_t G = q_heads / v->kv_heads;
    p.counter_bytes = 0;
    p.part_bytes = static_cast<uint64_t>(batch) * v->kv_heads * p.splits * record_floats(G, v->head_dim) * 4;
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

extern "C" miikv_status miikv_decode_attn(const miikv_view* view, const void* q, uint32_t q_dtype, uint32_t q_heads,
                                          float scale, uint32_t batch, const uint32_t* d_lengths,
                                          const miikv_decode_state* decode_state, uint32_t max_context, float* out,
                                          const float* gate, float* gated_out, void* workspace,
                                          uint64_t workspace_bytes, void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (q == nullptr || batch == 0 || q_heads == 0 || q_heads % view->kv_heads != 0 || !std::isfinite(scale))
        return MIIKV_EINVAL;
    const uint32_t G = q_heads / view->kv_heads;
    if (G > 16) return MIIKV_EUNSUPPORTED;
    if (q_dtype != MIIKV_DTYPE_F16 && q_dtype != MIIKV_DTYPE_F32) return MIIKV_EINVAL;
    if (out == nullptr && !(gate != nullptr && gated_out != nullptr)) return MIIKV_EINVAL;
    if ((gate == nullptr) != (gated_out == nullptr)) return MIIKV_EINVAL;
    if (d_lengths == nullptr && (decode_state == nullptr || batch != 1)) return MIIKV_EINVAL;
    if (max_context == 0 || max_context > view_seq_capacity(view)) return MIIKV_EINVAL;
    if (view->layout == MIIKV_LAYOUT_CONTIGUOUS && batch != 1) return MIIKV_EINVAL;
    const Plan p = make_plan(view, q_heads, batch, max_context);
    if (workspace == nullptr || workspace_bytes < p.counter_bytes + p.part_bytes) return MIIKV_EWORKSPACE;
    if (p.splits > 65535u || batch > 65535u || static_cast<uint64_t>(batch) * view->kv_heads > 0x7fffffffu)
        return MIIKV_EINVAL;

    DecodeArgs a;
    a.g = make_geo(*view);
    a.q = q;
    a.q_heads = q_heads;
    a.group = G;
    a.scale_log2 = scale * kLog2e;
    if (d_lengths != nullptr) {
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

    const size_t lds = (128 + kWavesPerWg * G * view->head_dim) * sizeof(float);
    if (lds > 64 * 1024) return MIIKV_EUNSUPPORTED;
    const dim3 grid(p.splits, view->kv_heads, batch);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool f32 = q_dtype == MIIKV_DTYPE_F32;
    const dim3 cgrid(batch * view->kv_heads, (G * view->head_dim + 63) / 64);
    if (view->head_dim == 128) {
        if (f32) hipLaunchKernelGGL((decode_kernel<128, true>), grid, dim3(256), lds, s, a);
        else hipLaunchKernelGGL((decode_kernel<128, false>), grid, dim3(256), lds, s, a);
        hipLaunchKernelGGL((combine_kernel<128>), cgrid, dim3(256), 0, s, a);
    } else {
        if (f32) hipLaunchKernelGGL((decode_kernel<256, true>), grid, dim3(256), lds, s, a);
        else hipLaunchKernelGGL((decode_kernel<256, false>), grid, dim3(256), lds, s, a);
        hipLaunchKernelGGL((combine_kernel<256>), cgrid, dim3(256), 0, s, a);
    }
    return hip_status(hipGetLastError());
}
