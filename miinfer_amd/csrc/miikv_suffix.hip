// Suffix (multi-token) attention over a cached q8_0 prefix on MFMA (gfx950).
//
// Token t of a T-token suffix sits at absolute position P + t and attends to
// cache positions [0, P + t]; the cache already holds the suffix's own rows
// (qwen3_primitives.hip:6826-6836).  For one kv head the query rows are the
// (token, head) pairs r = t*G + g; a workgroup owns 64 rows (four MFMA
// N-tiles, one per wave) and streams every key its rows can see.
//
// Each 32-key step is dequantised once per workgroup into fp16 tiles in LDS
// (double-buffered): K^[key][dim] = code * k_scale and V^[dim][key] =
// code * v_scale.  Per wave:
//   S^T[key][row] = K^_tile (16 keys x D) * Q^T (D x 16 rows)   v_mfma_f32_16x16x32_f16
//   O^T[dim][row] += V^T (16 dims x 16 keys) * P^T              v_mfma_f32_16x16x16_f16
// the S^T fragment being the P^T operand layout, as in the decode kernel.
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

constexpr uint32_t kSufRows = 64;      // query rows per workgroup
constexpr uint32_t kSufStep = 32;      // keys per step
constexpr float kLog2eS = 1.4426950408889634f;
constexpr float kSlackS = 6.0f;        // lazy-rescale threshold (log2 units): p <= 64
constexpr uint32_t kSufTargetWgs = 1024; // ~4 resident workgroups per CU over 256 CUs
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
    uint32_t splits;       // == gridDim.z
    float* part;           // partial records when splits > 1
    float* out;
    const float* gate;
    float* gated_out;
};

__device__ __forceinline__ float sfx_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// code * scale rounded once to fp16 (the code is exact in fp16), saturated to the
// finite range: 127 * fp16(amax / 127) can exceed 65504 for amax near the fp16 max.
template <typename V>
__device__ __forceinline__ V scale_sat(V codes, V scales) {
    const V lim = (V)(_Float16)65504.0f;
    return __builtin_elementwise_min(__builtin_elementwise_max(codes * scales, -lim), lim);
}

template <uint32_t D>
__global__ void __launch_bounds__(256) suffix_kernel(SuffixArgs a) {
    constexpr uint32_t NB = D / 32;
    constexpr uint32_t NM = D / 16;
    constexpr uint32_t KPAD = D + 8;        // K^ row stride (halves): staggers LDS banks
    constexpr uint32_t VPAD = kSufStep + 4; // V^ row stride (halves)
    constexpr uint32_t KCH = D / 128;       // 16-byte K chunks per thread per step
    constexpr uint32_t VCH = D / 64;        // 8-byte V chunks per thread per step
    __shared__ __align__(16) _Float16 s_k[2][kSufStep * KPAD];
    __shared__ __align__(16) _Float16 s_v[2][D * VPAD];
    __shared__ __align__(16) uint16_t s_ks[kSufStep * NB];   // [key][block]
    __shared__ __align__(16) uint16_t s_vs[NB * kSufStep];   // [block][key]

    const Geo& geo = a.g;
    uint32_t T = a.token_count;
    uint32_t P = a.base_position;
    if (a.ps != nullptr) {
        P = a.ps->base_position;
        T = min(T, a.ps->token_count);
    }
    const uint32_t G = a.group;
    const uint32_t h = blockIdx.y;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63;
    const uint32_t g4 = lane >> 4;
    const uint32_t n = lane & 15;
    const uint32_t rows = T * G;
    const uint32_t r0 = blockIdx.x * kSufRows;
    if (r0 >= rows) return;

    // This lane's query row (column n of its wave's N-tile).
    const uint32_t row = r0 + wave * 16 + n;
    const bool row_ok = row < rows;
    const uint32_t t_row = row_ok ? row / G : 0;
    const uint32_t qh = h * G + (row_ok ? row % G : 0);
    const uint32_t lim = P + t_row;  // last visible key (inclusive)

    // Keys the whole workgroup needs: up to the last row's limit.
    const uint32_t last_row = min(r0 + kSufRows, rows) - 1;
    const uint32_t nkeys = P + last_row / G + 1;
    const uint32_t split = blockIdx.z;
    const uint32_t key_lo = split * a.split_keys;
    if (key_lo >= nkeys) return;  // no row of this workgroup has keys in this split
    const uint32_t key_hi = min(nkeys, key_lo + a.split_keys);
    const uint32_t s_begin = key_lo / kSufStep;
    const uint32_t s_end = (key_hi + kSufStep - 1) / kSufStep;

    // ---- Q fragments (B operand): head qh of token t_row, dims 32*blk + 8*g4 .. +7.
    half8 qf[NB];
    {
        const size_t qrow = (static_cast<size_t>(t_row) * a.q_heads + qh) * D;
#pragma unroll
        for (uint32_t blk = 0; blk < NB; ++blk) {
            half8 v = {};
            if (row_ok) {
                if (a.q_f32) {
                    const float* qp = static_cast<const float*>(a.q) + qrow + blk * 32 + g4 * 8;
                    const float4 x0 = *reinterpret_cast<const float4*>(qp);
                    const float4 x1 = *reinterpret_cast<const float4*>(qp + 4);
                    v[0] = (_Float16)x0.x; v[1] = (_Float16)x0.y; v[2] = (_Float16)x0.z; v[3] = (_Float16)x0.w;
                    v[4] = (_Float16)x1.x; v[5] = (_Float16)x1.y; v[6] = (_Float16)x1.z; v[7] = (_Float16)x1.w;
                } else {
                    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qrow + blk * 32 + g4 * 8;
                    v = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(qp));
                }
            }
            qf[blk] = v;
        }
    }

    // ---- producer: global codes + scales of one step into registers
    const size_t slab_bytes = static_cast<size_t>(geo.page_tokens) * D;
    struct Stage {
        uint4 k[KCH];
        uint2 v[VCH];
        uint32_t ks, vs;  // two fp16 scales each (NB*32 halves per step over 256 threads)
    };
    auto load_stage = [&](uint32_t s, Stage& st) {
        const uint32_t tok0 = s * kSufStep;
        const size_t slab = slab_of(geo, a.seq, tok0, h);
        const uint32_t tp0 = tok0 % geo.page_tokens;
        const int8_t* kb = geo.k_codes + slab * slab_bytes + static_cast<size_t>(tp0) * D;
        const int8_t* vb = geo.v_codes + slab * slab_bytes + static_cast<size_t>(tp0) * D;
#pragma unroll
        for (uint32_t u = 0; u < KCH; ++u) st.k[u] = *reinterpret_cast<const uint4*>(kb + 16 * (tid + 256 * u));
#pragma unroll
        for (uint32_t u = 0; u < VCH; ++u) st.v[u] = *reinterpret_cast<const uint2*>(vb + 8 * (tid + 256 * u));
        const size_t sc0 = (slab * geo.page_tokens + tp0) * NB;  // 32*NB halves
        st.ks = st.vs = 0;
        if (tid < kSufStep * NB / 2) {
            st.ks = *reinterpret_cast<const uint32_t*>(geo.k_scales + sc0 + 2 * tid);
            st.vs = *reinterpret_cast<const uint32_t*>(geo.v_scales + sc0 + 2 * tid);
        }
    };
    // Scales to LDS (K as [key][block], V transposed to [block][key]).  Keys past the
    // cache end of this sequence get scale 0 so their (arbitrary) codes vanish.
    auto stage_scales = [&](uint32_t s, const Stage& st) {
        if (tid < kSufStep * NB / 2) {
            const uint32_t e0 = 2 * tid;            // element index key*NB + blk
            const uint32_t key = e0 / NB;
            const bool ok = s * kSufStep + key < nkeys;
            const uint32_t ks = ok ? st.ks : 0u, vs = ok ? st.vs : 0u;
            *reinterpret_cast<uint32_t*>(&s_ks[e0]) = ks;
            const uint32_t b0 = e0 % NB;
            s_vs[b0 * kSufStep + key] = static_cast<uint16_t>(vs & 0xffffu);
            s_vs[(b0 + 1) * kSufStep + key] = static_cast<uint16_t>(vs >> 16);
        }
    };
    // Dequantise the codes into fp16 tiles of buffer `buf`.
    auto stage_tiles = [&](uint32_t buf, const Stage& st) {
#pragma unroll
        for (uint32_t u = 0; u < KCH; ++u) {
            const uint32_t q = tid + 256 * u;              // 16-byte chunk of the 32*D K bytes
            const uint32_t T16 = q / D, qin = q % D;
            const uint32_t c = qin / 64, gq = (qin % 64) / 16, m = qin % 16;
            const uint32_t key = 16 * T16 + m;
            const uint32_t w[4] = {st.k[u].x, st.k[u].y, st.k[u].z, st.k[u].w};
#pragma unroll
            for (uint32_t e = 0; e < 2; ++e) {
                const uint32_t blk = 2 * c + e;
                const half8 scv = (half8)__builtin_bit_cast(_Float16, s_ks[key * NB + blk]);
                const half8 hv = scale_sat(codes8_to_half8(w[2 * e], w[2 * e + 1]), scv);
                *reinterpret_cast<half8*>(&s_k[buf][key * KPAD + 64 * c + 32 * e + 8 * gq]) = hv;
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < VCH; ++u) {
            const uint32_t q = tid + 256 * u;              // 8-byte chunk of the 32*D V bytes
            const uint32_t d = q / 4, Gq = q % 4;
            const uint32_t blk = d / 32;
            const uint32_t w[2] = {st.v[u].x, st.v[u].y};
#pragma unroll
            for (uint32_t J = 0; J < 2; ++J) {
                const half4 scv = *reinterpret_cast<const half4*>(&s_vs[blk * kSufStep + 16 * J + 4 * Gq]);
                const half4 hv = scale_sat(codes4_to_half4(w[J]), scv);
                *reinterpret_cast<half4*>(&s_v[buf][d * VPAD + 16 * J + 4 * Gq]) = hv;
            }
        }
    };

    float m_run = -INFINITY;
    float l_run = 0.0f;
    float4v O[NM];
#pragma unroll
    for (uint32_t mt = 0; mt < NM; ++mt) O[mt] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    Stage st;
    load_stage(s_begin, st);
    stage_scales(s_begin, st);
    __syncthreads();
    stage_tiles(s_begin & 1, st);
    __syncthreads();

    for (uint32_t s = s_begin; s < s_end; ++s) {
        const uint32_t buf = s & 1;
        const bool more = s + 1 < s_end;
        if (more) load_stage(s + 1, st);  // in flight during this step's MFMAs

        const uint32_t key0 = s * kSufStep;
        // Rows whose limit lies before this step skip its math (they are masked anyway).
        // ---- S^T for the two 16-key tiles
        float sc[2][4];
#pragma unroll
        for (uint32_t J = 0; J < 2; ++J) {
            float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t blk = 0; blk < NB; ++blk) {
                const half8 ka = *reinterpret_cast<const half8*>(&s_k[buf][(16 * J + n) * KPAD + 32 * blk + 8 * g4]);
                acc = mfma_16x16x32(ka, qf[blk], acc);
            }
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                const uint32_t key = key0 + 16 * J + 4 * g4 + i;
                sc[J][i] = (key <= lim && key < key_hi && row_ok) ? acc[i] * a.scale_log2 : -INFINITY;
            }
        }
        // ---- online softmax (per row n; lanes of the 4 groups share it)
        float cmax = sc[0][0];
#pragma unroll
        for (uint32_t J = 0; J < 2; ++J)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) cmax = fmaxf(cmax, sc[J][i]);
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
        const bool grow = cmax > m_run + kSlackS;
        if (__any(grow)) {
            const float m_new = grow ? cmax : m_run;
            const float alpha = sfx_exp2(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (uint32_t mt = 0; mt < NM; ++mt) O[mt] *= alpha;
        }
        // A row with no visible key yet keeps m_run = -inf; subtracting 0 keeps p = 0.
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        half4 pb[2];
#pragma unroll
        for (uint32_t J = 0; J < 2; ++J)
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {
                const float p = sfx_exp2(sc[J][i] - m_use);  // 0 for masked keys
                l_run += p;
                pb[J][i] = static_cast<_Float16>(p);
            }
        // ---- O^T += V^T * P^T
#pragma unroll
        for (uint32_t mt = 0; mt < NM; ++mt)
#pragma unroll
            for (uint32_t J = 0; J < 2; ++J) {
                const half4 va = *reinterpret_cast<const half4*>(&s_v[buf][(16 * mt + n) * VPAD + 16 * J + 4 * g4]);
                O[mt] = mfma_16x16x16(va, pb[J], O[mt]);
            }

        if (more) {
            stage_scales(s + 1, st);
            __syncthreads();   // scales visible; every wave is done with buffer buf^1's last use
            stage_tiles(buf ^ 1, st);
            __syncthreads();
        }
    }

    // ---- normalise and store: lane (g4, n) holds dims 16*mt + 4*g4 + i of row n.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (!row_ok) return;
    if (a.splits > 1) {
        // Partial record of (token t_row, kv head h, split): O [G][D], m [G], l [G].
        const uint32_t G_ = a.group;
        float* rec = a.part + ((static_cast<size_t>(t_row) * geo.kv_heads + h) * a.splits + split) *
                                  record_floats(G_, D);
        const uint32_t gi = qh - h * G_;
#pragma unroll
        for (uint32_t mt = 0; mt < NM; ++mt)
            *reinterpret_cast<float4*>(rec + gi * D + 16 * mt + 4 * g4) =
                make_float4(O[mt][0], O[mt][1], O[mt][2], O[mt][3]);
        if (g4 == 0) {
            rec[G_ * D + gi] = m_run;
            rec[G_ * D + G_ + gi] = l_run;
        }
        return;
    }
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    const size_t orow = (static_cast<size_t>(t_row) * a.q_heads + qh) * D;
#pragma unroll
    for (uint32_t mt = 0; mt < NM; ++mt) {
        float4 v;
        v.x = O[mt][0] * inv;
        v.y = O[mt][1] * inv;
        v.z = O[mt][2] * inv;
        v.w = O[mt][3] * inv;
        const size_t oi = orow + 16 * mt + 4 * g4;
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
    a.part = static_cast<float*>(workspace);
    a.out = out;
    a.gate = gate;
    a.gated_out = gated_out;
    const dim3 grid(static_cast<uint32_t>(blocks), view->kv_heads, plan.splits);
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
