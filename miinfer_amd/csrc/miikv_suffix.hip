// Suffix (multi-token) attention over a cached q8_0 prefix on MFMA (gfx950).
//
// Token t of a T-token suffix sits at absolute position P + t and attends to
// cache positions [0, P + t]; the cache already holds the suffix's own rows
// (qwen3_primitives.hip:6826-6836).  For one kv head the query rows are the
// (token, head) pairs r = t*G + g; a workgroup owns 128 rows (four waves of
// 32) and streams every key its rows can see.
//
// Each 32-key step is dequantised once per workgroup into fp16 tiles in LDS
// (double-buffered): K^[key][dim] = code * k_scale and V^T[dim][key] =
// code * v_scale, so every K/V byte read from HBM feeds 128 query rows and each
// LDS operand byte feeds 32.  The MFMAs are v_mfma_f32_32x32x16_f16.
// Online softmax in the log2 domain with a lazy running max.
//
// Split-K: grid.z cuts the key range into splits of a fixed number of keys so
// that a short suffix still fills the chip.  With one split the workgroup
// normalises and stores its rows; otherwise each (token, kv head, split) writes
// a partial record (unnormalised O, running max, sum) and the decode path's
// combine kernel merges them with token t's context length P + t + 1.
#include "miikv_common.hpp"
#include "miikv_split.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>

namespace miikv {

int validate_view(const miikv_view* v);
uint64_t view_seq_capacity(const miikv_view* v);

namespace {

constexpr uint32_t kSufRows = 128;     // query rows per workgroup (4 waves x 32)
constexpr uint32_t kSufStep = 32;      // keys per step
constexpr float kLog2eS = 1.4426950408889634f;
constexpr float kSlackS = 6.0f;        // lazy-rescale threshold (log2 units): p <= 64
constexpr uint32_t kSufTargetWgs = 1024; // ~4 workgroups per CU over 256 CUs
constexpr uint32_t kSufMaxSplits = 64;

struct SuffixArgs {
    Geo g;
    const void* q;
    uint32_t q_f32;
    uint32_t q_heads;
    uint32_t group;
    float scale_log2;
    uint32_t token_count;  // host upper bound
    uint32_t base_position;
    uint32_t seq;
    const miikv_prefill_state* ps;
    uint32_t split_keys;   // keys per split (multiple of kSufStep)
    uint32_t splits;
    uint32_t row_blocks;   // workgroups per (kv head, split) group
    float* part;           // partial records when splits > 1
    float* out;
    const float* gate;
    float* gated_out;
};

__device__ __forceinline__ float sfx_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Largest fp16 scale whose product with any code (|code| <= 128) stays finite:
// 128 * 511.75 = 65504.  Scales above it only arise for blocks whose absmax is
// within 0.8% of the fp16 maximum; clamping them bounds the tile to finite values.
constexpr float kMaxTileScale = 511.75f;

__device__ __forceinline__ half2v clamp_scales(uint32_t bits) {
    const half2v lim = {(_Float16)kMaxTileScale, (_Float16)kMaxTileScale};
    return __builtin_elementwise_min(__builtin_bit_cast(half2v, bits), lim);
}

// The two MFMAs of the step loop, written out so that register classes are fixed:
// the loop-invariant query fragments (QK B operand) live in accumulation
// registers, which leaves the 256 architectural VGPRs to the O^T accumulators
// (128 registers at D = 256), the staging, LDS fragments and softmax.  The
// compiler does not see these as MFMAs, so each carries its own wait states: a
// VALU write read by an MFMA needs 2 (the leading s_nop; when the MFMA unit is
// busy with the previous MFMA it costs nothing), MFMAs accumulating into the same
// registers back to back need none, and an MFMA result read by VALU needs 18
// (mfma_result_wait).
__device__ __forceinline__ void mfma_qk(half8 k, half8 q_agpr, float16v& s) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(s) : "v"(k), "a"(q_agpr));
}
__device__ __forceinline__ void mfma_pv(half8 v, half8 p, float16v& o) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(o) : "v"(v), "v"(p));
}
__device__ __forceinline__ void mfma_result_wait(float16v& c) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3" : "+v"(c));
}

// Workgroup: 4 waves x 32 query rows.  Per 32-key step and wave (32x32x16 MFMAs):
//   S^T[key][row] (32x32) = sum over D/16 dim chunks of K^[key][16 dims] * Q^T
//   O^T[dim][row] += V^T[32 dims][16 keys] * P^T, two key halves per 32-dim tile
// The S^T accumulator of lane (n = lane % 32, hh = lane / 32) holds row n and keys
// 8j + 4hh + i (register 4j + i); the B operand of the PV MFMA for key half kc
// is registers 8kc .. 8kc+7, provided V^T's key order within a half is permuted
// the same way: LDS position 8*b2 + 4*b3 + i holds key 8*b3 + 4*b2 + i.
//
// One barrier per step: during step s the waves run the MFMAs of step s from LDS
// buffer s&1 while dequantising step s+1 (codes fetched during step s-1) into
// buffer (s+1)&1 and fetching step s+2.  V scales are staged transposed in LDS
// one step ahead; K scales are read per chunk straight from global memory.
template <uint32_t D>
__global__ void __launch_bounds__(256) suffix_kernel(SuffixArgs a) {
    constexpr uint32_t NB = D / 32;         // q8_0 blocks per row = PV M-tiles
    constexpr uint32_t NC = D / 16;         // QK k-chunks
    constexpr uint32_t KPAD = D + 8;        // K^ row stride (halves)
    constexpr uint32_t VPAD = kSufStep + 8; // V^T row stride (halves)
    constexpr uint32_t KCH = D / 128;       // 16-byte K chunks per thread per step
    constexpr uint32_t VCH = D / 128;       // 16-byte V chunks per thread per step
    __shared__ __align__(16) _Float16 s_k[2][kSufStep * KPAD];
    __shared__ __align__(16) _Float16 s_v[2][D * VPAD];
    __shared__ __align__(16) _Float16 s_vs[2][NB * kSufStep];  // [block][key]

    const Geo& geo = a.g;
    uint32_t T = a.token_count;
    uint32_t P = a.base_position;
    if (a.ps != nullptr) {
        P = a.ps->base_position;
        T = min(T, a.ps->token_count);
    }
    const uint32_t G = a.group;
    // XCD-aware order: workgroup L runs on XCD L % 8, so the row blocks of one
    // (kv head, split) group, which read the same K/V tiles, are given to one XCD
    // and share its L2.  Groups g = xcd, xcd + 8, ...; the grid is padded to a
    // multiple of 8 groups.
    const uint32_t L = blockIdx.x;
    const uint32_t j = L / 8;
    const uint32_t grp = (L % 8) + 8 * (j / a.row_blocks);
    if (grp >= a.g.kv_heads * a.splits) return;
    const uint32_t h = grp % a.g.kv_heads;
    const uint32_t split = grp / a.g.kv_heads;
    const uint32_t rb = j % a.row_blocks;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63;
    const uint32_t n = lane & 31;
    const uint32_t hh = lane >> 5;
    const uint32_t rows = T * G;
    const uint32_t r0 = rb * kSufRows;
    if (r0 >= rows) return;

    const uint32_t row = r0 + wave * 32 + n;
    const bool row_ok = row < rows;
    const uint32_t t_row = row_ok ? row / G : 0;
    const uint32_t qh = h * G + (row_ok ? row % G : 0);
    const uint32_t lim = P + t_row;  // last visible key (inclusive)
    // Smallest limit among this wave's rows: steps wholly at or below it need no mask.
    const uint32_t wave_lim = P + min(r0 + wave * 32, rows - 1) / G;

    const uint32_t last_row = min(r0 + kSufRows, rows) - 1;
    const uint32_t nkeys = P + last_row / G + 1;
    const uint32_t key_lo = split * a.split_keys;
    if (key_lo >= nkeys) return;  // no row of this workgroup has keys in this split
    const uint32_t key_hi = min(nkeys, key_lo + a.split_keys);
    const uint32_t s_begin = key_lo / kSufStep;
    const uint32_t s_end = (key_hi + kSufStep - 1) / kSufStep;

    // ---- Q^T fragments (B operand): row n, dims 16c + 8hh .. +7.
    half8 qf[NC];
    {
        const size_t qrow = (static_cast<size_t>(t_row) * a.q_heads + qh) * D;
#pragma unroll
        for (uint32_t c = 0; c < NC; ++c) {
            half8 v = {};
            if (row_ok) {
                if (a.q_f32) {
                    const float* qp = static_cast<const float*>(a.q) + qrow + c * 16 + hh * 8;
                    const float4 x0 = *reinterpret_cast<const float4*>(qp);
                    const float4 x1 = *reinterpret_cast<const float4*>(qp + 4);
                    v[0] = (_Float16)x0.x; v[1] = (_Float16)x0.y; v[2] = (_Float16)x0.z; v[3] = (_Float16)x0.w;
                    v[4] = (_Float16)x1.x; v[5] = (_Float16)x1.y; v[6] = (_Float16)x1.z; v[7] = (_Float16)x1.w;
                } else {
                    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qrow + c * 16 + hh * 8;
                    v = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(qp));
                }
            }
            qf[c] = v;
        }
    }

    // ---- producer: codes and scales of one step into registers.
    const size_t slab_bytes = static_cast<size_t>(geo.page_tokens) * D;
    struct Stage {
        uint32_t ks[KCH];   // K scales of the chunk's two blocks
        uint4 k[KCH];
        uint4 v[VCH];
    };
    auto slab_at = [&](uint32_t s) { return slab_of(geo, a.seq, s * kSufStep, h); };
    auto scale_base = [&](uint32_t s, size_t slab) {
        return (slab * geo.page_tokens + (s * kSufStep) % geo.page_tokens) * NB;
    };
    auto code_base = [&](uint32_t s, size_t slab) {
        return slab * slab_bytes + static_cast<size_t>((s * kSufStep) % geo.page_tokens) * D;
    };
    // Two V scales per thread (key = 2*tid / NB, blocks 2*tid % NB and +1).
    auto load_vs = [&](uint32_t s, size_t slab) -> uint32_t {
        if (tid >= kSufStep * NB / 2) return 0u;
        return *reinterpret_cast<const uint32_t*>(geo.v_scales + scale_base(s, slab) + 2 * tid);
    };
    auto load_k = [&](uint32_t s, size_t slab, Stage& st) {
        const size_t sc0 = scale_base(s, slab);
        const int8_t* kb = geo.k_codes + code_base(s, slab);
#pragma unroll
        for (uint32_t u = 0; u < KCH; ++u) {
            const uint32_t q = tid + 256 * u;
            const uint32_t key = 16 * (q / D) + q % 16;
            const uint32_t c = (q % D) / 64;
            st.ks[u] = *reinterpret_cast<const uint32_t*>(geo.k_scales + sc0 + key * NB + 2 * c);
            st.k[u] = *reinterpret_cast<const uint4*>(kb + 16 * q);
        }
    };
    auto load_v = [&](uint32_t s, size_t slab, Stage& st) {
        const int8_t* vb = geo.v_codes + code_base(s, slab);
#pragma unroll
        for (uint32_t u = 0; u < VCH; ++u) st.v[u] = *reinterpret_cast<const uint4*>(vb + 16 * (tid + 256 * u));
    };
    // V scales of step s into s_vs[buf] ([block][key]); keys at or past key_hi get 0
    // so their codes (possibly never written) contribute nothing.
    auto write_vs = [&](uint32_t s, uint32_t vs, uint32_t buf) {
        if (tid < kSufStep * NB / 2) {
            const uint32_t e0 = 2 * tid;
            const uint32_t key = e0 / NB;
            const uint32_t b0 = e0 % NB;
            const half2v sc = s * kSufStep + key < key_hi ? clamp_scales(vs) : half2v{};
            s_vs[buf][b0 * kSufStep + key] = sc[0];
            s_vs[buf][(b0 + 1) * kSufStep + key] = sc[1];
        }
    };
    // K^ tile: chunk q = key 16*(q/D) + q%16, dims 64c + 8g + j (block 2c) and
    // 64c + 32 + 8g + j (block 2c+1).
    auto dequant_k = [&](const Stage& st, uint32_t buf) {
#pragma unroll
        for (uint32_t u = 0; u < KCH; ++u) {
            const uint32_t q = tid + 256 * u;
            const uint32_t qin = q % D;
            const uint32_t c = qin / 64, g = (qin % 64) / 16;
            const uint32_t key = 16 * (q / D) + q % 16;
            const half2v sc = clamp_scales(st.ks[u]);
            const half8 lo = codes8_to_half8(st.k[u].x, st.k[u].y) * (half8)sc[0];
            const half8 hi = codes8_to_half8(st.k[u].z, st.k[u].w) * (half8)sc[1];
            _Float16* dst = &s_k[buf][key * KPAD + 64 * c + 8 * g];
            *reinterpret_cast<half8*>(dst) = lo;
            *reinterpret_cast<half8*>(dst + 32) = hi;
        }
    };
    // V^T tile: chunk q = dim q/2, 16 bytes at 16*(q%2) of the dim's 32 codes:
    // dwords hold keys 8u+0..3, 16+8u+0..3, 8u+4..7, 16+8u+4..7 (u = q%2).
    auto dequant_v = [&](const Stage& st, uint32_t buf) {
#pragma unroll
        for (uint32_t u = 0; u < VCH; ++u) {
            const uint32_t q = tid + 256 * u;
            const uint32_t d = q / 2, up = q % 2;
            const _Float16* sv = &s_vs[buf][(d / 32) * kSufStep];
            const half8 slo = *reinterpret_cast<const half8*>(sv + 8 * up);
            const half8 shi = *reinterpret_cast<const half8*>(sv + 16 + 8 * up);
            const half4 a0 = codes4_to_half4(st.v[u].x) * slo.lo;
            const half4 a1 = codes4_to_half4(st.v[u].y) * shi.lo;
            const half4 a2 = codes4_to_half4(st.v[u].z) * slo.hi;
            const half4 a3 = codes4_to_half4(st.v[u].w) * shi.hi;
            _Float16* dst = &s_v[buf][d * VPAD + 4 * up];
            *reinterpret_cast<half4*>(dst) = a0;
            *reinterpret_cast<half4*>(dst + 16) = a1;
            *reinterpret_cast<half4*>(dst + 8) = a2;
            *reinterpret_cast<half4*>(dst + 24) = a3;
        }
    };

    float m_run = -INFINITY;
    float l_run = 0.0f;
    float16v O[NB];
#pragma unroll
    for (uint32_t mt = 0; mt < NB; ++mt) O[mt] = float16v{};

    // Prologue: step s_begin dequantised, step s_begin+1 codes in registers and its
    // V scales in LDS, step s_begin+2's V scales in a register.
    Stage st;
    size_t slab = slab_at(s_begin);
    load_k(s_begin, slab, st);
    load_v(s_begin, slab, st);
    write_vs(s_begin, load_vs(s_begin, slab), s_begin & 1);
    __syncthreads();
    dequant_k(st, s_begin & 1);
    dequant_v(st, s_begin & 1);
    if (s_begin + 1 < s_end) {
        slab = slab_at(s_begin + 1);
        load_k(s_begin + 1, slab, st);
        load_v(s_begin + 1, slab, st);
        write_vs(s_begin + 1, load_vs(s_begin + 1, slab), (s_begin + 1) & 1);
    }
    size_t slab2 = 0;   // slab of step s+2
    uint32_t vs2 = 0;   // V scales of step s+2
    if (s_begin + 2 < s_end) {
        slab2 = slab_at(s_begin + 2);
        vs2 = load_vs(s_begin + 2, slab2);
    }
    __syncthreads();

    for (uint32_t s = s_begin; s < s_end; ++s) {
        const uint32_t buf = s & 1;
        const bool next = s + 1 < s_end;
        const bool next2 = s + 2 < s_end;
        const bool next3 = s + 3 < s_end;
        // ---- S^T = K^ Q^T
        float16v acc = {};
        const _Float16* kt = &s_k[buf][n * KPAD + 8 * hh];
        mfma_qk(*reinterpret_cast<const half8*>(kt), qf[0], acc);
#pragma unroll
        for (uint32_t c = 1; c < NC; ++c) mfma_qk(*reinterpret_cast<const half8*>(kt + 16 * c), qf[c], acc);
        mfma_result_wait(acc);
        if (next) dequant_k(st, buf ^ 1);
        if (next2) load_k(s + 2, slab2, st);
        size_t slab3 = 0;
        uint32_t vs3 = 0;
        if (next3) {
            slab3 = slab_at(s + 3);
            vs3 = load_vs(s + 3, slab3);
        }

        // ---- online softmax over this lane's 16 keys of row n
        const uint32_t key0 = s * kSufStep;
        if (key0 + kSufStep - 1 > wave_lim || key0 + kSufStep > key_hi) {
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) {
                const uint32_t key = key0 + 8 * (r / 4) + 4 * hh + (r % 4);
                if (!(key <= lim && key < key_hi)) acc[r] = -INFINITY;
            }
        }
        float cmax = acc[0];
#pragma unroll
        for (uint32_t r = 1; r < 16; ++r) cmax = fmaxf(cmax, acc[r]);
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
        const float cm = cmax * a.scale_log2;
        const bool grow = cm > m_run + kSlackS;
        if (__any(grow)) {
            const float m_new = grow ? cm : m_run;
            const float alpha = sfx_exp2(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (uint32_t mt = 0; mt < NB; ++mt) O[mt] *= alpha;
        }
        // A row with no visible key yet keeps m_run = -inf; subtracting 0 keeps p = 0.
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        half8 pb[2];
#pragma unroll
        for (uint32_t kc = 0; kc < 2; ++kc)
#pragma unroll
            for (uint32_t e = 0; e < 8; e += 2) {
                const float p0 = sfx_exp2(fmaf(acc[8 * kc + e], a.scale_log2, -m_use));
                const float p1 = sfx_exp2(fmaf(acc[8 * kc + e + 1], a.scale_log2, -m_use));
                l_run += p0 + p1;
                pb[kc][e] = static_cast<_Float16>(p0);  // round to nearest: no bias against l_run
                pb[kc][e + 1] = static_cast<_Float16>(p1);
            }
        // ---- O^T += V^T P^T
        const _Float16* vt = &s_v[buf][n * VPAD + 8 * hh];
        mfma_pv(*reinterpret_cast<const half8*>(vt), pb[0], O[0]);
        mfma_pv(*reinterpret_cast<const half8*>(vt + 16), pb[1], O[0]);
#pragma unroll
        for (uint32_t mt = 1; mt < NB; ++mt)
#pragma unroll
            for (uint32_t kc = 0; kc < 2; ++kc)
                mfma_pv(*reinterpret_cast<const half8*>(vt + 32 * mt * VPAD + 16 * kc), pb[kc], O[mt]);
        if (next) dequant_v(st, buf ^ 1);
        if (next2) {
            load_v(s + 2, slab2, st);
            write_vs(s + 2, vs2, buf);
        }
        slab2 = slab3;
        vs2 = vs3;
        __syncthreads();
    }

#pragma unroll
    for (uint32_t mt = 0; mt < NB; ++mt) mfma_result_wait(O[mt]);
    // ---- store: lane (n, hh) holds dims 32mt + 8j + 4hh + i of row n (register 4j + i).
    l_run += __shfl_xor(l_run, 32, 64);
    if (!row_ok) return;
    if (a.splits > 1) {
        // Partial record of (token t_row, kv head h, split): O [G][D], m [G], l [G].
        float* rec = a.part + ((static_cast<size_t>(t_row) * geo.kv_heads + h) * a.splits + split) *
                                  record_floats(G, D);
        const uint32_t gi = qh - h * G;
#pragma unroll
        for (uint32_t mt = 0; mt < NB; ++mt)
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j)
                *reinterpret_cast<float4*>(rec + gi * D + 32 * mt + 8 * j + 4 * hh) =
                    make_float4(O[mt][4 * j], O[mt][4 * j + 1], O[mt][4 * j + 2], O[mt][4 * j + 3]);
        if (hh == 0) {
            rec[G * D + gi] = m_run;
            rec[G * D + G + gi] = l_run;
        }
        return;
    }
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const size_t orow = (static_cast<size_t>(t_row) * a.q_heads + qh) * D;
#pragma unroll
    for (uint32_t mt = 0; mt < NB; ++mt)
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            float4 v;
            v.x = O[mt][4 * j] * inv;
            v.y = O[mt][4 * j + 1] * inv;
            v.z = O[mt][4 * j + 2] * inv;
            v.w = O[mt][4 * j + 3] * inv;
            const size_t oi = orow + 32 * mt + 8 * j + 4 * hh;
            if (a.out) *reinterpret_cast<float4*>(a.out + oi) = v;
            if (a.gate && a.gated_out) {
                const float4 gv = *reinterpret_cast<const float4*>(a.gate + oi);
                float4 r;
                r.x = v.x * (1.0f / (1.0f + expf(-gv.x)));
                r.y = v.y * (1.0f / (1.0f + expf(-gv.y)));
                r.z = v.z * (1.0f / (1.0f + expf(-gv.z)));
                r.w = v.w * (1.0f / (1.0f + expf(-gv.w)));
                *reinterpret_cast<float4*>(a.gated_out + oi) = r;
            }
        }
}

}  // namespace
}  // namespace miikv

using namespace miikv;

namespace {

struct SuffixPlan {
    uint32_t splits;
    uint32_t split_keys;
    uint64_t part_bytes;
};

// Split count for a suffix of `tokens` tokens whose keys end at or before
// `key_bound`: enough workgroups to fill the chip, at least 256 keys per split.
// Monotone in key_bound, so a plan made with the cache capacity covers any
// smaller context.
SuffixPlan make_suffix_plan(const miikv_view* v, uint32_t q_heads, uint32_t tokens, uint64_t key_bound) {
    SuffixPlan p{1, 0, 0};
    const uint32_t G = q_heads / v->kv_heads;
    const uint64_t wgs = (static_cast<uint64_t>(tokens) * G + kSufRows - 1) / kSufRows * v->kv_heads;
    uint64_t want = (kSufTargetWgs + wgs - 1) / wgs;
    if (const char* e = std::getenv("MIIKV_SUFFIX_SPLITS")) want = std::strtoul(e, nullptr, 10);
    const uint64_t by_keys = (key_bound + 255) / 256;
    want = std::min<uint64_t>({want, by_keys, kSufMaxSplits});
    if (want <= 1) return p;
    const uint64_t unit = kWavesPerWg * kChunk;  // the combine's split granularity (128 keys)
    const uint64_t cpw = (key_bound + want * unit - 1) / (want * unit);
    p.split_keys = static_cast<uint32_t>(cpw * unit);
    p.splits = static_cast<uint32_t>((key_bound + p.split_keys - 1) / p.split_keys);
    if (p.splits <= 1) return SuffixPlan{1, 0, 0};
    p.part_bytes = static_cast<uint64_t>(tokens) * v->kv_heads * p.splits * record_floats(G, v->head_dim) * 4;
    return p;
}

}  // namespace

// Workspace for the split-K path: partial records of every (token, kv head, split),
// planned for the cache capacity (any base position fits).  0 when one split suffices.
extern "C" uint64_t miikv_suffix_workspace_bytes(const miikv_view* view, uint32_t q_heads, uint32_t token_count) {
    if (validate_view(view) != MIIKV_OK || q_heads == 0 || q_heads % view->kv_heads != 0 || token_count == 0)
        return 0;
    return make_suffix_plan(view, q_heads, token_count, view_seq_capacity(view)).part_bytes;
}

extern "C" miikv_status miikv_suffix_attn(const miikv_view* view, const void* q, uint32_t q_dtype, uint32_t q_heads,
                                          float scale, uint32_t token_count, uint32_t base_position, uint32_t seq,
                                          const miikv_prefill_state* prefill_state, float* out, const float* gate,
                                          float* gated_out, void* workspace, uint64_t workspace_bytes,
                                          void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (q == nullptr || q_heads == 0 || q_heads % view->kv_heads != 0 || !std::isfinite(scale)) return MIIKV_EINVAL;
    if (q_dtype != MIIKV_DTYPE_F16 && q_dtype != MIIKV_DTYPE_F32) return MIIKV_EINVAL;
    const uint32_t G = q_heads / view->kv_heads;
    if (out == nullptr && !(gate != nullptr && gated_out != nullptr)) return MIIKV_EINVAL;
    if ((gate == nullptr) != (gated_out == nullptr)) return MIIKV_EINVAL;
    if (view->layout == MIIKV_LAYOUT_CONTIGUOUS && seq != 0) return MIIKV_EINVAL;
    if (token_count == 0) return MIIKV_OK;
    const uint64_t cap = view_seq_capacity(view);
    if (prefill_state == nullptr && static_cast<uint64_t>(base_position) + token_count > cap) return MIIKV_EINVAL;
    const uint64_t rows = static_cast<uint64_t>(token_count) * G;
    const uint64_t blocks = (rows + kSufRows - 1) / kSufRows;
    if (blocks > 0x7fffffffu || static_cast<uint64_t>(token_count) * view->kv_heads > 0x7fffffffu)
        return MIIKV_EINVAL;
    // Without a workspace the kernel runs one split; with one, the plan for the
    // known context (host base position) or for the capacity (device state).
    SuffixPlan plan{1, 0, 0};
    if (workspace != nullptr) {
        const uint64_t bound = prefill_state ? cap : static_cast<uint64_t>(base_position) + token_count;
        plan = make_suffix_plan(view, q_heads, token_count, bound);
        if (workspace_bytes < plan.part_bytes) return MIIKV_EWORKSPACE;
    }
    SuffixArgs a;
    a.g = make_geo(*view);
    a.q = q;
    a.q_f32 = q_dtype == MIIKV_DTYPE_F32;
    a.q_heads = q_heads;
    a.group = G;
    a.scale_log2 = scale * kLog2eS;
    a.token_count = token_count;
    a.base_position = base_position;
    a.seq = seq;
    a.ps = prefill_state;
    a.split_keys = plan.splits > 1 ? plan.split_keys : 0xffffffffu;
    a.splits = plan.splits;
    a.row_blocks = static_cast<uint32_t>(blocks);
    a.part = static_cast<float*>(workspace);
    a.out = out;
    a.gate = gate;
    a.gated_out = gated_out;
    const uint64_t groups = static_cast<uint64_t>(view->kv_heads) * plan.splits;
    const uint64_t wgs = ((groups + 7) / 8) * 8 * blocks;
    if (wgs > 0x7fffffffu) return MIIKV_EINVAL;
    const dim3 grid(static_cast<uint32_t>(wgs));
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (view->head_dim == 128) hipLaunchKernelGGL(suffix_kernel<128>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(suffix_kernel<256>, grid, dim3(256), 0, s, a);
    if (plan.splits > 1) {
        // Token t of the suffix sees P + t + 1 keys; rows past the device token count are skipped.
        SplitArgs c{};
        c.g = a.g;
        c.q_heads = q_heads;
        c.group = G;
        c.len_ptr = prefill_state ? &prefill_state->base_position : nullptr;
        c.len_stride = 0;
        c.len_add = (prefill_state ? 0u : base_position) + 1u;
        c.len_bstep = 1;
        c.count_ptr = prefill_state ? &prefill_state->token_count : nullptr;
        c.max_context = static_cast<uint32_t>(std::min<uint64_t>(cap, 0xffffffffu));
        c.cpw = plan.split_keys / (kWavesPerWg * kChunk);
        c.max_splits = plan.splits;
        c.part = a.part;
        c.out = out;
        c.gate = gate;
        c.gated_out = gated_out;
        const dim3 cgrid(token_count * view->kv_heads, (G * view->head_dim + 63) / 64);
        if (view->head_dim == 128) hipLaunchKernelGGL(combine_kernel<128>, cgrid, dim3(256), 0, s, c);
        else hipLaunchKernelGGL(combine_kernel<256>, cgrid, dim3(256), 0, s, c);
    }
    return hip_status(hipGetLastError());
}
