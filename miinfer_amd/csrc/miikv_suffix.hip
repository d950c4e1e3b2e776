// Suffix (multi-token) attention over a cached q8_0 prefix on MFMA (gfx950).
//
// Token t of a T-token suffix sits at absolute position P + t and attends to
// cache positions [0, P + t]; the cache already holds the suffix's own rows
// (qwen3_primitives.hip:6826-6836).  For one kv head the query rows are the
// (token, head) pairs r = t*G + g.
//
// Two kernels (plus the split combine):
//  1. expand_kernel dequantises every 32-key step of the context once into
//     fp16 tiles in the workspace, laid out as the MFMA operand fragments the
//     attention waves read: K^ = code * k_scale as the A operand of S^T = K^ Q^T,
//     V^T = code * v_scale as the A operand of O^T += V^T P^T.  Each K/V byte is
//     dequantised once instead of once per row block.  With the fused append it
//     also quantises and stores the suffix's own rows.
//  2. suffix_kernel: a workgroup owns 32 query rows per wave and streams the
//     fp16 tiles of its key range through LDS (direct global->LDS loads, four
//     buffers, prefetch two steps ahead, one barrier per step).  Per 32-key step and wave
//     (v_mfma_f32_32x32x16_f16):
//        S^T[key][row] (32x32) = sum over D/16 dim chunks of K^[32 keys][16] Q^T
//        O^T[dim][row]        += V^T[32 dims][16 keys] P^T, two key halves per tile
//     The S^T accumulator of lane (n = lane % 32, hh = lane / 32) holds row n
//     and keys 8j + 4hh + i (register 4j + i); registers 8kc..8kc+7 form the B
//     operand of the PV MFMA for key half kc, given that V^T's key order within
//     a half is permuted alike: fragment position 4*b3 + i of lane hh holds key
//     8*b3 + 4*hh + i.  Online softmax in the log2 domain with a lazy max.
//
// Split-K: the key range is cut into splits of a fixed number of keys so that
// a short suffix still fills the chip.  With one split the workgroup normalises
// and stores its rows; otherwise each (token, kv head, split) writes a partial
// record (unnormalised O, running max, sum) and suffix_combine_kernel merges
// them with token t's context length P + t + 1.
#include "miikv_suffix.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>

namespace miikv {

int validate_view(const miikv_view* v);
uint64_t view_seq_capacity(const miikv_view* v);

namespace {

// Largest fp16 scale whose product with any code (|code| <= 128) stays finite:
// 128 * 511.75 = 65504.  Scales above it only arise for blocks whose absmax is
// within 0.8% of the fp16 maximum; clamping them keeps the tiles finite.
constexpr float kMaxTileScale = 511.75f;

__device__ __forceinline__ _Float16 clamp_scale(uint16_t bits) {
    return __builtin_elementwise_min(__builtin_bit_cast(_Float16, bits), (_Float16)kMaxTileScale);
}

// Keys of the context: [0, P + T).
__device__ __forceinline__ uint32_t context_keys(uint32_t host_count, const miikv_prefill_state* ps) {
    return ps ? min(host_count, ps->base_position + ps->token_count) : host_count;
}

// One 32-key step of kv head blockIdx.y: 256 threads; keys at or past the context
// end become 0 (their codes may never have been written).
// Fused append (APPEND, a.k_new set): a step holding any of the suffix's own keys
// [P, P + T) first assembles its 32-token group in LDS -- the cached codes and
// scales of the other keys, the suffix rows quantised with the append rule (the
// bytes miikv_append_f16 stores) -- writes the whole group back to the cache with
// 16-byte stores and expands it from LDS.
template <uint32_t D, bool APPEND>
__global__ void __launch_bounds__(256) expand_kernel(ExpandArgs a) {
    constexpr uint32_t NB = D / 32;
    constexpr uint32_t NKF = D / 16;       // K fragments per step
    constexpr uint32_t PER = D / 64;       // fragment lanes per thread, per operand
    __shared__ __align__(16) _Float16 s_vs[NB * kSufStep];  // [block][key]
    __shared__ __align__(16) uint8_t s_grp[APPEND ? 2 * kSufStep * D + 2 * kSufStep * NB * 2 : 16];
    const Geo& geo = a.g;
    // Last step first: with the fused append the suffix's steps, which carry the
    // longer quantise-and-store chain, are dispatched ahead of the rest.
    const uint32_t step = a.step0 + (gridDim.x - 1 - blockIdx.x);
    const uint32_t h = blockIdx.y;
    const uint32_t tid = threadIdx.x;
    const uint32_t nkeys = context_keys(a.key_count, a.ps);
    const uint32_t tok0 = step * kSufStep;
    if (tok0 >= nkeys) return;
    if (a.current && a.ps != nullptr && step < a.ps->base_position / kSufStep) return;  // already expanded
    const size_t slab = slab_of(geo, a.seq, tok0, h);
    const uint32_t tp0 = tok0 % geo.page_tokens;
    const size_t sc0 = (slab * geo.page_tokens + tp0) * NB;
    const size_t cb = slab * static_cast<size_t>(geo.page_tokens) * D + static_cast<size_t>(tp0) * D;
    const int8_t* kb = geo.k_codes + cb;
    const int8_t* vb = geo.v_codes + cb;
    // fp16 planes (the control path): the tiles are the stored fp16 rows themselves
    const _Float16* kb16 = reinterpret_cast<const _Float16*>(geo.k_codes) + cb;
    const _Float16* vb16 = reinterpret_cast<const _Float16*>(geo.v_codes) + cb;
    const uint16_t* ksc = geo.k_scales + sc0;
    const uint16_t* vsc = geo.v_scales + sc0;
    if constexpr (APPEND) {
        const uint32_t P = a.ps ? a.ps->base_position : a.base_position;
        const uint32_t T = a.ps ? min(a.token_count, a.ps->token_count) : a.token_count;
        if (tok0 + kSufStep > P && tok0 < P + T) {
            // The suffix rows of this step, thread (key tl, 16-dim chunk q16) per item,
            // loaded first so that they travel with the cached group below.
            constexpr uint32_t ITEMS = kSufStep * (D / 16) / 256;
            uint4 rk[ITEMS][2], rv[ITEMS][2];
#pragma unroll
            for (uint32_t it = 0; it < ITEMS; ++it) {
                const uint32_t w = tid + 256 * it, tl = w / (D / 16), q16 = w % (D / 16);
                const uint32_t key = tok0 + tl;
                const uint32_t t = key >= P && key < P + T ? key - P : 0;
                const size_t src = (static_cast<size_t>(t) * geo.kv_heads + h) * D + q16 * 16;
                rk[it][0] = *reinterpret_cast<const uint4*>(a.k_new + src);
                rk[it][1] = *reinterpret_cast<const uint4*>(a.k_new + src + 8);
                rv[it][0] = *reinterpret_cast<const uint4*>(a.v_new + src);
                rv[it][1] = *reinterpret_cast<const uint4*>(a.v_new + src + 8);
            }
            // Group in LDS: [K codes 32*D][V codes 32*D][K scales 32*NB][V scales 32*NB]
            // in the cache's slab order.  Copy the cached group (its keys outside the
            // suffix keep their bytes), then overwrite the suffix keys.
            uint4* g16 = reinterpret_cast<uint4*>(s_grp);
            constexpr uint32_t CK = kSufStep * D / 16, CS = kSufStep * NB * 2 / 16;
            for (uint32_t c = tid; c < 2 * CK + 2 * CS; c += 256) {
                const uint4* src = c < CK ? reinterpret_cast<const uint4*>(kb) + c
                                 : c < 2 * CK ? reinterpret_cast<const uint4*>(vb) + (c - CK)
                                 : c < 2 * CK + CS ? reinterpret_cast<const uint4*>(ksc) + (c - 2 * CK)
                                                   : reinterpret_cast<const uint4*>(vsc) + (c - 2 * CK - CS);
                g16[c] = *src;
            }
            __syncthreads();
            uint8_t* s_k = s_grp;
            uint8_t* s_v = s_grp + kSufStep * D;
            uint16_t* s_ks = reinterpret_cast<uint16_t*>(s_grp + 2 * kSufStep * D);
            uint16_t* s_vsc = s_ks + kSufStep * NB;
            // partner lanes q16 ^ 1 hold the two halves of a 32-value block
#pragma unroll
            for (uint32_t it = 0; it < ITEMS; ++it) {
                const uint32_t w = tid + 256 * it, tl = w / (D / 16), q16 = w % (D / 16);
                const uint32_t key = tok0 + tl;
                const bool mine = key >= P && key < P + T;
                float xk[16], xv[16];
                unpack16_f16(rk[it], xk);
                unpack16_f16(rv[it], xv);
                int8_t qk[16], qv[16];
                float sk, sv;
                quantize16(xk, qk, sk);  // both lanes of a pair reach the shuffles
                quantize16(xv, qv, sv);
                if (!mine) continue;
                const uint32_t d0 = q16 * 16;
                uint32_t packed[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    packed[u] = static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * u])) |
                                (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * u + 1])) << 8) |
                                (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * u + 2])) << 16) |
                                (static_cast<uint32_t>(static_cast<uint8_t>(qk[4 * u + 3])) << 24);
                *reinterpret_cast<uint2*>(s_k + k_code_offset(tl, d0, D)) = make_uint2(packed[0], packed[1]);
                *reinterpret_cast<uint2*>(s_k + k_code_offset(tl, d0 + 8, D)) = make_uint2(packed[2], packed[3]);
#pragma unroll
                for (int u = 0; u < 16; ++u) s_v[v_code_offset(tl, d0 + u, D)] = static_cast<uint8_t>(qv[u]);
                if ((q16 & 1) == 0) {
                    s_ks[tl * NB + d0 / 32] = f32_to_f16_bits(sk);
                    s_vsc[tl * NB + d0 / 32] = f32_to_f16_bits(sv);
                }
            }
            __syncthreads();
            for (uint32_t c = tid; c < 2 * CK + 2 * CS; c += 256) {
                uint4* dst = c < CK ? reinterpret_cast<uint4*>(geo.k_codes + cb) + c
                           : c < 2 * CK ? reinterpret_cast<uint4*>(geo.v_codes + cb) + (c - CK)
                           : c < 2 * CK + CS ? reinterpret_cast<uint4*>(geo.k_scales + sc0) + (c - 2 * CK)
                                             : reinterpret_cast<uint4*>(geo.v_scales + sc0) + (c - 2 * CK - CS);
                *dst = g16[c];
            }
            kb = reinterpret_cast<const int8_t*>(s_k);
            vb = reinterpret_cast<const int8_t*>(s_v);
            ksc = s_ks;
            vsc = s_vsc;
        }
    }
    if (tid < kSufStep * NB && !geo.v_f16) {
        const uint32_t key = tid / NB, blk = tid % NB;
        s_vs[blk * kSufStep + key] = tok0 + key < nkeys ? clamp_scale(vsc[tid]) : (_Float16)0.0f;
    }
    __syncthreads();
    _Float16* out = a.tiles + (static_cast<size_t>(h) * a.steps + step) * tile_halves(D);
    // K fragment c, lane (n, hh): key n, dims 16c + 8hh .. +7.  In the cache tile
    // those 8 codes sit at (key/16)*16D + (c/4)*1024 + g*256 + (key%16)*16 + e*8
    // with e = (c%4)/2, g = 2*(c%2) + hh.
#pragma unroll
    for (uint32_t u = 0; u < PER; ++u) {
        const uint32_t fl = tid + 256 * u;
        const uint32_t c = fl / 64, l = fl % 64, n = l % 32, hh = l / 32;
        const uint32_t off = (n / 16) * 16 * D + (c / 4) * 1024 + (2 * (c % 2) + hh) * 256 + (n % 16) * 16 +
                             ((c % 4) / 2) * 8;
        if (geo.k_f16) {
            const half8 x = *reinterpret_cast<const half8*>(kb16 + off);
            *reinterpret_cast<half8*>(out + 8 * fl) = tok0 + n < nkeys ? x : half8{};
            continue;
        }
        const uint2 w = *reinterpret_cast<const uint2*>(kb + off);
        const _Float16 sc = tok0 + n < nkeys ? clamp_scale(ksc[n * NB + c / 2]) : (_Float16)0.0f;
        *reinterpret_cast<half8*>(out + 8 * fl) = codes8_to_half8(w.x, w.y) * (half8)sc;
    }
    // V fragment f = 2mt + kc, lane (n, hh): dim 32mt + n, positions 4*b3 + i hold
    // keys 16kc + 8*b3 + 4hh + i.  A 32-token group stores dim d's code of key
    // 16J + 4G + I at d*32 + 8G + 4J + I, so b3 = 0 is the dword at G = hh and
    // b3 = 1 the dword at G = 2 + hh, both at J = kc.
#pragma unroll
    for (uint32_t u = 0; u < PER; ++u) {
        const uint32_t fl = tid + 256 * u;
        const uint32_t f = fl / 64, l = fl % 64, n = l % 32, hh = l / 32;
        const uint32_t mt = f / 2, kc = f % 2;
        if (geo.v_f16) {
            const _Float16* vd16 = vb16 + (32 * mt + n) * 32;
            half4 a0 = *reinterpret_cast<const half4*>(vd16 + 8 * hh + 4 * kc);
            half4 a1 = *reinterpret_cast<const half4*>(vd16 + 8 * (2 + hh) + 4 * kc);
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i) {  // keys 16kc + 4hh + i and 16kc + 8 + 4hh + i
                if (tok0 + 16 * kc + 4 * hh + i >= nkeys) a0[i] = (_Float16)0.0f;
                if (tok0 + 16 * kc + 8 + 4 * hh + i >= nkeys) a1[i] = (_Float16)0.0f;
            }
            half8 r;
            r.lo = a0;
            r.hi = a1;
            *reinterpret_cast<half8*>(out + 64 * 8 * NKF + 8 * fl) = r;
            continue;
        }
        const int8_t* vd = vb + (32 * mt + n) * 32;
        const uint32_t w0 = *reinterpret_cast<const uint32_t*>(vd + 8 * hh + 4 * kc);
        const uint32_t w1 = *reinterpret_cast<const uint32_t*>(vd + 8 * (2 + hh) + 4 * kc);
        const _Float16* sv = &s_vs[mt * kSufStep + 16 * kc + 4 * hh];
        const half4 a0 = codes4_to_half4(w0) * *reinterpret_cast<const half4*>(sv);
        const half4 a1 = codes4_to_half4(w1) * *reinterpret_cast<const half4*>(sv + 8);
        half8 r;
        r.lo = a0;
        r.hi = a1;
        *reinterpret_cast<half8*>(out + 64 * 8 * NKF + 8 * fl) = r;
    }
}

// This file is compiled with MFMA results in architectural VGPRs
// (-amdgpu-mfma-vgpr-form): at D = 256 a wave holds O^T (128 registers), the
// query fragments (64), S^T (16) and the softmax working set, and within the 256
// registers of two waves per SIMD the lazy rescale multiplies O^T in place.
#ifndef MIIKV_SUFFIX_STAGGER
#define MIIKV_SUFFIX_STAGGER 1
#endif
constexpr bool kSufStagger = MIIKV_SUFFIX_STAGGER != 0;
// Prefetch distance in steps (config 4, same box: 1 and 3 both ~1-2 us slower
// than 2; 3 takes all 160 KB of LDS).
#ifndef MIIKV_SUFFIX_DIST
#define MIIKV_SUFFIX_DIST 2
#endif
constexpr uint32_t kDist = MIIKV_SUFFIX_DIST;
constexpr uint32_t kSufBufs = kSufStagger ? kDist + 2 : kDist + 1;  // LDS tile buffers


// The softmax keeps its VALU count low (v_max3 row max, v_dot2 row sum): VALU work
// of the two waves of a SIMD hides only partly under their MFMAs.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float max3_raw(float x, float y, float z) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(y), "v"(z));
    return r;
}

template <uint32_t D>
__global__ void __launch_bounds__(64 * kSufWaves) suffix_kernel(SuffixArgs a) {
    constexpr uint32_t NB = D / 32;         // PV M-tiles
    constexpr uint32_t NC = D / 16;         // QK k-chunks (K fragments)
    constexpr uint32_t TILE = tile_halves(D);
    constexpr uint32_t CHUNKS = TILE * 2 / 1024;  // 1 KiB copy chunks per step
    static_assert(CHUNKS % kSufWaves == 0, "copy chunks must split evenly over waves");
    __shared__ __align__(16) _Float16 s_t[kSufBufs][TILE];
    // The tile buffers are the kernel's whole LDS.  Measured at D = 256: 8 bytes of
    // LDS beyond 128 KiB (two flags) slowed the step loop by ~12%, so any other LDS
    // variable has to live inside these buffers.
    static_assert(sizeof(s_t) <= 128u * 1024u, "suffix LDS must stay within 128 KiB");

    uint32_t T = a.token_count;
    uint32_t P = a.base_position;
    if (a.ps != nullptr) {
        P = a.ps->base_position;
        T = min(T, a.ps->token_count);
    }
    const uint32_t G = a.group;
    // XCD-aware order: workgroup L runs on XCD L % 8.  Each XCD gets an equal,
    // contiguous range of the (group, row block) sequence, group-major, so the
    // row blocks of one (kv head, split) group, which read the same tiles, share
    // an L2; with rows_together the sequence is (kv head, row block, split).  The
    // grid is padded to a multiple of 8 workgroups.
    const uint32_t L = blockIdx.x;
    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t idx = (L % 8) * per_xcd + L / 8;
    uint32_t h, split, rb;
    if (a.rows_together) {
        // the splits of one row block next to each other: an XCD's workgroups share
        // their query rows through its L2 (and each tile range among fewer of them)
        const uint32_t gi = idx / a.splits;
        split = idx % a.splits;
        h = gi / a.row_blocks;
        rb = gi % a.row_blocks;
        if (h >= a.g.kv_heads) return;
    } else {
        const uint32_t grp = idx / a.row_blocks;
        if (grp >= a.g.kv_heads * a.splits) return;
        h = grp % a.g.kv_heads;
        split = grp / a.g.kv_heads;
        rb = idx % a.row_blocks;
    }
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
        const size_t qrow = (static_cast<size_t>(t_row) * a.q_heads + qh) * D;  // a valid row also when !row_ok
        if (a.q_f32) {
            // Batches of four fragments, loaded without a branch and then converted: a
            // per-fragment load in a branch was waited for at the branch's end, one
            // round trip per fragment.
#pragma unroll
            for (uint32_t c0 = 0; c0 < NC; c0 += 4) {
                float4 x[4][2];
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) {
                    const float* qp = static_cast<const float*>(a.q) + qrow + (c0 + j) * 16 + hh * 8;
                    x[j][0] = *reinterpret_cast<const float4*>(qp);
                    x[j][1] = *reinterpret_cast<const float4*>(qp + 4);
                }
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) {
                    half8 v;
                    v[0] = (_Float16)x[j][0].x; v[1] = (_Float16)x[j][0].y; v[2] = (_Float16)x[j][0].z; v[3] = (_Float16)x[j][0].w;
                    v[4] = (_Float16)x[j][1].x; v[5] = (_Float16)x[j][1].y; v[6] = (_Float16)x[j][1].z; v[7] = (_Float16)x[j][1].w;
                    qf[c0 + j] = row_ok ? v : half8{};
                }
            }
        } else {
            // every load issued unconditionally (qrow is a valid row), then selected
#pragma unroll
            for (uint32_t c = 0; c < NC; ++c) {
                const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qrow + c * 16 + hh * 8;
                qf[c] = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(qp));
            }
#pragma unroll
            for (uint32_t c = 0; c < NC; ++c) qf[c] = row_ok ? qf[c] : half8{};
        }
    }

    // Step s's tile into LDS buffer b: CHUNKS KiB, each wave copying every
    // kSufWaves-th KiB with one 16-byte direct-to-LDS load per lane.
    const char* tiles_h = reinterpret_cast<const char*>(a.tiles + static_cast<size_t>(h) * a.steps * TILE);
    auto fetch = [&](uint32_t s, uint32_t b) {
        const char* src = tiles_h + static_cast<size_t>(s) * TILE * 2 + lane * 16;
        char* dst = reinterpret_cast<char*>(s_t[b]);
#pragma unroll
        for (uint32_t u = 0; u < CHUNKS / kSufWaves; ++u) {
            const uint32_t chunk = wave + kSufWaves * u;
            __builtin_amdgcn_global_load_lds(src + chunk * 1024, dst + chunk * 1024, 16, 0, 0);
        }
    };

    float m_run = -INFINITY;
    float l_run = 0.0f;
    float16v O[NB];
#pragma unroll
    for (uint32_t mt = 0; mt < NB; ++mt) O[mt] = float16v{};

    // Step s lives in buffer s % kSufBufs; the fetch of step s + kDist is issued at
    // the top of step s into a buffer that no wave reads any more (the barrier that
    // ends each step orders it after those reads).
    constexpr uint32_t kPer = CHUNKS / kSufWaves;  // loads per wave per fetch
    for (uint32_t k = 0; k < kDist; ++k)
        if (s_begin + k < s_end) fetch(s_begin + k, (s_begin + k) % kSufBufs);
    // the query and the first step's tile; the later prefetches may stay in flight
    if (kDist > 1 && s_begin + 1 < s_end) wait_vmem_le<(kDist - 1) * kPer>();
    else wait_vmem();
    __syncthreads();

    // ---- S^T = K^ Q^T of step s
    auto scores = [&](uint32_t s) __attribute__((always_inline)) {
        const _Float16* tk = s_t[s % kSufBufs] + lane * 8;
        float16v acc = {};
#pragma unroll
        for (uint32_t c = 0; c < NC; ++c) acc = mfma_32x32x16(*reinterpret_cast<const half8*>(tk + 512 * c), qf[c], acc);
        return acc;
    };
    // ---- online softmax over this lane's 16 keys of row n; P^T fragments out
    auto softmax = [&](uint32_t s, float16v acc, half8 (&pb)[2]) __attribute__((always_inline)) {
        const uint32_t key0 = s * kSufStep;
        if (key0 + kSufStep - 1 > wave_lim || key0 + kSufStep > key_hi) {
#pragma unroll
            for (uint32_t r = 0; r < 16; ++r) {
                const uint32_t key = key0 + 8 * (r / 4) + 4 * hh + (r % 4);
                if (!(key <= lim && key < key_hi)) acc[r] = -INFINITY;
            }
        }
        // v_max3 straight on the MFMA results: fmaxf would first quieten each input
        // (one more v_max per element), and the scores hold no NaN.
        const float t0 = max3_raw(acc[0], acc[1], acc[2]), t1 = max3_raw(acc[3], acc[4], acc[5]);
        const float t2 = max3_raw(acc[6], acc[7], acc[8]), t3 = max3_raw(acc[9], acc[10], acc[11]);
        const float t4 = max3_raw(acc[12], acc[13], acc[14]);
        float cmax = max3_raw(max3_raw(t0, t1, t2), max3_raw(t3, t4, acc[15]), -INFINITY);
        cmax = swap32_reduce(cmax, MaxOp{});
        const float cm = cmax * a.scale_log2;
        const bool grow = cm > m_run + kSlackS;
        if (__any(grow)) {
            const float m_new = grow ? cm : m_run;
            const float alpha = grow ? sfx_exp2(m_run - cm) : 1.0f;  // (-inf - -inf would be NaN)
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (uint32_t mt = 0; mt < NB; ++mt) O[mt] *= alpha;
        }
        // A row with no visible key yet keeps m_run = -inf; subtracting 0 keeps p = 0.
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        // l sums the fp16 weights the PV MFMAs use, two per v_dot2 (fp32 accumulation).
#pragma unroll
        for (uint32_t kc = 0; kc < 2; ++kc)
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e)
                pb[kc][e] = static_cast<_Float16>(sfx_exp2(fmaf(acc[8 * kc + e], a.scale_log2, -m_use)));
        const half2v one2 = {(_Float16)1.0f, (_Float16)1.0f};
        float ls0 = 0.0f, ls1 = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            ls0 = __builtin_amdgcn_fdot2(half2v{pb[0][2 * j], pb[0][2 * j + 1]}, one2, ls0, false);
            ls1 = __builtin_amdgcn_fdot2(half2v{pb[1][2 * j], pb[1][2 * j + 1]}, one2, ls1, false);
        }
        l_run += ls0 + ls1;
    };
    // ---- O^T += V^T P^T of step s
    auto values = [&](uint32_t s, const half8 (&pb)[2]) __attribute__((always_inline)) {
        const _Float16* tv = s_t[s % kSufBufs] + 64 * 8 * NC + lane * 8;
#pragma unroll
        for (uint32_t mt = 0; mt < NB; ++mt)
#pragma unroll
            for (uint32_t kc = 0; kc < 2; ++kc)
                O[mt] = mfma_32x32x16(*reinterpret_cast<const half8*>(tv + 512 * (2 * mt + kc)), pb[kc], O[mt]);
    };
    // Top of step s: the fetch of step s + kDist.  End of step s: step s+1's tile
    // must have landed (this step's own fetch may stay in flight), then the barrier.
    auto step_begin = [&](uint32_t s) __attribute__((always_inline)) {
        if (s + kDist < s_end) fetch(s + kDist, (s + kDist) % kSufBufs);
    };
    auto step_end = [&](uint32_t s) __attribute__((always_inline)) {
        if (s + kDist < s_end) wait_vmem_le<(kDist > 1 ? kPer : 0)>();
        else wait_vmem();
        __syncthreads();
    };

    // With kSufStagger the two waves of each SIMD (waves w and w + kSufWaves/2)
    // run half a step apart: the leading half orders a step as scores, softmax,
    // values; the lagging half adds step s-1's values before step s's scores, so
    // one wave's softmax can overlap the other's MFMAs (C4: ~2% faster).
    // Every wave still passes one barrier per step; the lagging half's values of
    // step s-1 read a buffer that is refilled only at the top of step s+1
    // (kSufBufs >= kDist + 2).
    const bool lag = kSufStagger && wave >= kSufWaves / 2;
    if (!lag) {
        for (uint32_t s = s_begin; s < s_end; ++s) {
            step_begin(s);
            half8 pb[2];
            softmax(s, scores(s), pb);
            values(s, pb);
            step_end(s);
        }
    } else {
        half8 pprev[2];
        step_begin(s_begin);
        softmax(s_begin, scores(s_begin), pprev);
        step_end(s_begin);
        for (uint32_t s = s_begin + 1; s < s_end; ++s) {
            step_begin(s);
            values(s - 1, pprev);
            softmax(s, scores(s), pprev);
            step_end(s);
        }
        values(s_end - 1, pprev);
    }

    // ---- store: lane (n, hh) holds dims 32mt + 8j + 4hh + i of row n (register 4j + i).
    l_run = swap32_reduce(l_run, AddOp{});
    if (!row_ok) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    if (a.splits > 1) {
        const uint32_t rows_cap = a.token_count * G;
        const size_t pr = (static_cast<size_t>(split) * a.g.kv_heads + h) * rows_cap + row;
        _Float16* po = static_cast<_Float16*>(a.part) + pr * D;
#pragma unroll
        for (uint32_t mt = 0; mt < NB; ++mt)
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                half4 v;
#pragma unroll
                for (uint32_t i = 0; i < 4; ++i) v[i] = static_cast<_Float16>(O[mt][4 * j + i] * inv);
                *reinterpret_cast<half4*>(po + 32 * mt + 8 * j + 4 * hh) = v;
            }
        if (hh == 0) {
            float2* ml = reinterpret_cast<float2*>(static_cast<_Float16*>(a.part) +
                                                   part_o_halves(a.splits, a.g.kv_heads, rows_cap, D));
            ml[pr] = make_float2(m_run, l_run);
        }
        return;
    }
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

// ---- exact products on MFMA (MIIKV_SUFFIX_EXACT for long suffixes) -------------
//
// The reference multiplies an fp32 query with the dequantised keys in fp32.  Here the
// scores are exact in the same sense as decode's: the key tiles hold the int8 codes
// as fp16 (exact), each 32-value block's dot product comes out of its own
// v_mfma_f32_16x16x32_f16 (16 keys x 16 query rows) and is multiplied by the block's
// fp16 scale in fp32, and an fp32 query is split into fp16 hi + lo parts with a second
// MFMA per block for the lo part.  The values enter as their codes (fp16, exact), and
// each block's scale multiplies the probabilities in fp32, the product rounded to
// fp16 once, as on the decode path; O^T += V^T P^T runs as v_mfma_f32_16x16x32_f16,
// one per 16 dims with the P^T of their block.  A wave serves 16 query rows and holds
// the query's hi and lo parts (64 registers) and O^T (64 registers).
//
// Step record of the exact tiles (halves):
//   K codes as fp16 [2 key tiles t][D/32 blocks b][64 lanes][8]: lane (g, i) = 16g + i
//     holds key 16t + i, dims 32b + 8g .. +7 (the A operand of the score MFMA);
//   K block scales [t][4 g][D/32 b][4 r]: the scale of key 16t + 4g + r, block b (the
//     keys a score lane holds);
//   V block scales [D/32 b][4 g][8 e]: the scale of key ex_key(g, e), block b (0 past
//     the context end);
//   V^T codes as fp16 [D/16 dim tiles m][64 lanes][8]: lane (g, i) holds dim 16m + i
//     of keys ex_key(g, e), e < 8.
// ex_key(g, e) is the key in score register e % 4 of tile e / 4 of lane group g, so a
// lane's eight probabilities are directly its PV B operand.
__host__ __device__ constexpr uint32_t ex_tile_halves(uint32_t D) { return 64 * D + 64 * (D / 32); }
__device__ __forceinline__ uint32_t ex_key(uint32_t g, uint32_t e) { return 16 * (e >> 2) + 4 * g + (e & 3); }

// One 32-key step of kv head blockIdx.y into the exact tile layout (q8 planes only);
// keys at or past the context end get zero codes and scales.
template <uint32_t D>
__global__ void __launch_bounds__(256) expand_exact_kernel(ExpandArgs a) {
    constexpr uint32_t NB = D / 32;
    constexpr uint32_t PER = D / 64;  // fragment lanes per thread, per operand
    __shared__ __align__(16) _Float16 s_vs[NB * kSufStep];  // [block][key]
    const Geo& geo = a.g;
    const uint32_t step = a.step0 + blockIdx.x;
    const uint32_t h = blockIdx.y;
    const uint32_t tid = threadIdx.x;
    const uint32_t nkeys = context_keys(a.key_count, a.ps);
    const uint32_t tok0 = step * kSufStep;
    if (tok0 >= nkeys) return;
    const size_t slab = slab_of(geo, a.seq, tok0, h);
    const uint32_t tp0 = tok0 % geo.page_tokens;
    const size_t sc0 = (slab * geo.page_tokens + tp0) * NB;
    const size_t cb = slab * static_cast<size_t>(geo.page_tokens) * D + static_cast<size_t>(tp0) * D;
    const int8_t* kb = geo.k_codes + cb;
    const int8_t* vb = geo.v_codes + cb;
    const uint16_t* ksc = geo.k_scales + sc0;
    const uint16_t* vsc = geo.v_scales + sc0;
    if (tid < kSufStep * NB) {
        const uint32_t key = tid / NB, blk = tid % NB;
        s_vs[blk * kSufStep + key] = tok0 + key < nkeys ? __builtin_bit_cast(_Float16, vsc[tid]) : (_Float16)0.0f;
    }
    __syncthreads();
    _Float16* out = a.tiles + (static_cast<size_t>(h) * a.steps + step) * ex_tile_halves(D);
    // K codes: fragment (t, b), lane (g, i): key 16t + i, dims 32b + 8g .. +7, which sit
    // in the cache tile at t*16D + (b/2)*1024 + g*256 + i*16 + (b%2)*8
#pragma unroll
    for (uint32_t u = 0; u < PER; ++u) {
        const uint32_t fl = tid + 256 * u;
        const uint32_t f = fl / 64, l = fl % 64, g = l / 16, i = l % 16;
        const uint32_t t = f / NB, b = f % NB;
        const uint32_t off = t * 16 * D + (b / 2) * 1024 + g * 256 + i * 16 + (b % 2) * 8;
        const uint2 w = *reinterpret_cast<const uint2*>(kb + off);
        *reinterpret_cast<half8*>(out + 8 * fl) = tok0 + 16 * t + i < nkeys ? codes8_to_half8(w.x, w.y) : half8{};
    }
    // K scales [t][g][b][r] = scale of key 16t + 4g + r, block b (raw fp16)
    _Float16* osc = out + 32 * D;
    if (tid < 32 * NB) {
        const uint32_t t = tid / (16 * NB), g = (tid / (4 * NB)) % 4, b = (tid / 4) % NB, r = tid % 4;
        const uint32_t key = 16 * t + 4 * g + r;
        osc[tid] = tok0 + key < nkeys ? __builtin_bit_cast(_Float16, ksc[key * NB + b]) : (_Float16)0.0f;
    }
    // V scales [b][g][e] = scale of key ex_key(g, e), block b (0 past the context)
    _Float16* ovs = osc + 32 * NB;
    if (tid < 32 * NB) {
        const uint32_t b = tid / 32, g = (tid / 8) & 3, e = tid & 7;
        ovs[tid] = s_vs[b * kSufStep + ex_key(g, e)];
    }
    // V^T code fragments: dim tile m, lane (g, i): dim 16m + i, keys ex_key(g, 0..7) =
    // 4g .. 4g+3 and 16 + 4g .. 16 + 4g + 3, i.e. (J = 0, G = g) and (J = 1, G = g) in
    // the cache group's order (code of key 16J + 4G + I of dim d at d*32 + 8G + 4J + I):
    // eight contiguous bytes.  Codes past the context end are read as they are: their
    // scale is 0.
    _Float16* ov = ovs + 32 * NB;
#pragma unroll
    for (uint32_t u = 0; u < PER; ++u) {
        const uint32_t fl = tid + 256 * u;
        const uint32_t m = fl / 64, l = fl % 64, g = l / 16, i = l % 16;
        const uint2 w = *reinterpret_cast<const uint2*>(vb + (16 * m + i) * 32 + 8 * g);
        *reinterpret_cast<half8*>(ov + 8 * fl) = codes8_to_half8(w.x, w.y);
    }
}

// Two fp16 products (p0 * lo half of w, p1 * hi half of w), each of an fp32 value and
// an fp16 value rounded to fp16 once (v_fma_mix with a zero addend), packed in one word.
__device__ __forceinline__ uint32_t mul_round2(float p0, float p1, uint32_t w) {
    uint32_t d;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]\n\t"
        "v_fma_mixhi_f16 %0, %3, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
        : "=&v"(d)
        : "v"(p0), "v"(w), "v"(p1));
    return d;
}

#ifndef MIIKV_EXACT_WAVES
#define MIIKV_EXACT_WAVES 8
#endif
constexpr uint32_t kExWaves = MIIKV_EXACT_WAVES;
constexpr uint32_t kExRows = 16 * kExWaves;  // query rows per workgroup
constexpr uint32_t kExDist = 2;              // prefetch distance in steps
constexpr uint32_t kExBufs = kExDist + 1;    // LDS step buffers

template <uint32_t D, bool QF32>
__global__ void __launch_bounds__(64 * kExWaves) suffix_exact_kernel(SuffixArgs a) {
    constexpr uint32_t NB = D / 32;          // q8 blocks
    constexpr uint32_t NM = D / 16;          // PV dim tiles
    constexpr uint32_t REC = ex_tile_halves(D);
    constexpr uint32_t KV_CHUNKS = 64 * D * 2 / 1024;  // 1 KiB chunks of K codes + V^T
    constexpr uint32_t kChunkLoads = (KV_CHUNKS + kExWaves - 1) / kExWaves;  // per wave (the last maybe empty)
    constexpr uint32_t kPer = kChunkLoads + 1;  // loads per wave per fetch (+1: the scales)
    constexpr uint32_t SC_PIECES = 128 * NB / 16;  // 16-byte scale pieces of a step
    constexpr uint32_t SC_LANES = (SC_PIECES + kExWaves - 1) / kExWaves;  // per wave
    __shared__ __align__(16) _Float16 s_t[kExBufs][REC];
    static_assert(sizeof(s_t) <= 128u * 1024u, "exact suffix LDS must stay within 128 KiB");

    uint32_t T = a.token_count;
    uint32_t P = a.base_position;
    if (a.ps != nullptr) {
        P = a.ps->base_position;
        T = min(T, a.ps->token_count);
    }
    const uint32_t G = a.group;
    const uint32_t L = blockIdx.x;
    const uint32_t per_xcd = gridDim.x / 8;
    const uint32_t idx = (L % 8) * per_xcd + L / 8;
    const uint32_t grp = idx / a.row_blocks;
    if (grp >= a.g.kv_heads * a.splits) return;
    const uint32_t h = grp % a.g.kv_heads;
    const uint32_t split = grp / a.g.kv_heads;
    const uint32_t rb = idx % a.row_blocks;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint32_t lane = tid & 63;
    const uint32_t ci = lane & 15;  // the lane's row (column of every MFMA)
    const uint32_t gq = lane >> 4;  // lane group: keys 4gq .. +3 of each 16-key tile
    const uint32_t rows = T * G;
    const uint32_t r0 = rb * kExRows;
    if (r0 >= rows) return;

    const uint32_t row = r0 + wave * 16 + ci;
    const bool row_ok = row < rows;
    const uint32_t t_row = row_ok ? row / G : 0;
    const uint32_t qh = h * G + (row_ok ? row % G : 0);
    const uint32_t lim = P + t_row;  // last visible key (inclusive) of this lane's row
    const uint32_t wave_lim = P + min(r0 + wave * 16, rows - 1) / G;

    const uint32_t last_row = min(r0 + kExRows, rows) - 1;
    const uint32_t nkeys = P + last_row / G + 1;
    const uint32_t key_lo = split * a.split_keys;
    if (key_lo >= nkeys) return;
    const uint32_t key_hi = min(nkeys, key_lo + a.split_keys);
    const uint32_t s_begin = key_lo / kSufStep;
    const uint32_t s_end = (key_hi + kSufStep - 1) / kSufStep;

    // ---- Q^T fragments (B operand of the score MFMA): row ci, dims 32b + 8gq .. +7;
    // an fp32 query as hi + lo parts
    half8 qhi[NB];
    half8 qlo[QF32 ? NB : 1];
    {
        const size_t qrow = (static_cast<size_t>(t_row) * a.q_heads + qh) * D;
        if constexpr (QF32) {
#pragma unroll
            for (uint32_t b0 = 0; b0 < NB; b0 += 4) {
                float4 x[4][2];
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) {
                    const float* qp = static_cast<const float*>(a.q) + qrow + (b0 + j) * 32 + gq * 8;
                    x[j][0] = *reinterpret_cast<const float4*>(qp);
                    x[j][1] = *reinterpret_cast<const float4*>(qp + 4);
                }
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j) {
                    const float xs[8] = {x[j][0].x, x[j][0].y, x[j][0].z, x[j][0].w,
                                         x[j][1].x, x[j][1].y, x[j][1].z, x[j][1].w};
                    half8 hi8, lo8;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const _Float16 hv = static_cast<_Float16>(xs[e]);
                        hi8[e] = hv;
                        lo8[e] = static_cast<_Float16>(xs[e] - static_cast<float>(hv));
                    }
                    qhi[b0 + j] = row_ok ? hi8 : half8{};
                    qlo[b0 + j] = row_ok ? lo8 : half8{};
                }
            }
        } else {
#pragma unroll
            for (uint32_t b = 0; b < NB; ++b) {
                const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qrow + b * 32 + gq * 8;
                const half8 v = __builtin_bit_cast(half8, *reinterpret_cast<const uint4*>(qp));
                qhi[b] = row_ok ? v : half8{};
            }
        }
    }

    const char* tiles_h = reinterpret_cast<const char*>(a.tiles + static_cast<size_t>(h) * a.steps * REC);
    auto fetch = [&](uint32_t s, uint32_t b) {
        const char* src = tiles_h + static_cast<size_t>(s) * REC * 2;
        char* dst = reinterpret_cast<char*>(s_t[b]);
        // K codes (32*D halves) and V^T codes (32*D halves) as 1 KiB chunks, and the K and
        // V scales between them (128*NB bytes) as 16-byte pieces, SC_LANES per wave
        // Every wave issues kPer loads, so that the wait counts below hold for every wave:
        // a load past the step's chunks (or pieces) repeats one in range into that one's
        // own place (the same bytes twice).
#pragma unroll
        for (uint32_t u = 0; u < kChunkLoads; ++u) {
            const uint32_t chunk = min(wave + kExWaves * u, KV_CHUNKS - 1);
            const uint32_t off = chunk < KV_CHUNKS / 2 ? chunk * 1024 : chunk * 1024 + 128 * NB;
            __builtin_amdgcn_global_load_lds(src + off + lane * 16, dst + off, 16, 0, 0);
        }
        const uint32_t soff = 64 * D + min(wave * SC_LANES, SC_PIECES - SC_LANES) * 16;
        if (lane < SC_LANES) __builtin_amdgcn_global_load_lds(src + soff + lane * 16, dst + soff, 16, 0, 0);
    };

    float m_run = -INFINITY;
    float l_run = 0.0f;
    float4v O[NM];
#pragma unroll
    for (uint32_t m = 0; m < NM; ++m) O[m] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    for (uint32_t k = 0; k < kExDist; ++k)
        if (s_begin + k < s_end) fetch(s_begin + k, (s_begin + k) % kExBufs);
    wait_vmem();
    __syncthreads();

    // One step; MASK: the step holds keys past some row's limit or past the split.
    auto step = [&](uint32_t s, auto mask_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
        if (s + kExDist < s_end) fetch(s + kExDist, (s + kExDist) % kExBufs);
        const _Float16* tb = s_t[s % kExBufs];
        // ---- scores of the lane's 8 keys (tile t, keys 16t + 4gq + r): one MFMA per q8
        // block (two with a lo part), the block scale applied in fp32
        float pf[8];
#pragma unroll
        for (uint32_t t = 0; t < 2; ++t) {
            const _Float16* tk = tb + t * NB * 512 + lane * 8;
            const _Float16* tsc = tb + 32 * D + (t * 4 + gq) * 4 * NB;
            float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (uint32_t b = 0; b < NB; ++b) {
                const half8 kf = *reinterpret_cast<const half8*>(tk + 512 * b);
                float4v c = mfma_16x16x32(kf, qhi[b], float4v{0.0f, 0.0f, 0.0f, 0.0f});
                if constexpr (QF32) c = mfma_16x16x32(kf, qlo[b], c);
                const half4 sc = *reinterpret_cast<const half4*>(tsc + 4 * b);
#pragma unroll
                for (uint32_t r = 0; r < 4; ++r) acc[r] = fmaf(c[r], static_cast<float>(sc[r]), acc[r]);
            }
#pragma unroll
            for (uint32_t r = 0; r < 4; ++r) pf[4 * t + r] = acc[r];
        }
        // ---- mask and online softmax: the row's 32 keys sit in the 4 lanes of its column
        if constexpr (MASK) {
            const uint32_t key0 = s * kSufStep;
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e) {
                const uint32_t key = key0 + ex_key(gq, e);
                if (!(key <= lim && key < key_hi)) pf[e] = -INFINITY;
            }
        }
        float cmax = fmaxf(fmaxf(fmaxf(pf[0], pf[1]), fmaxf(pf[2], pf[3])), fmaxf(fmaxf(pf[4], pf[5]), fmaxf(pf[6], pf[7])));
        cmax = rows_reduce(cmax, MaxOp{});
        const float cm = cmax * a.scale_log2;
        const bool grow = cm > m_run + kSlackS;
        if (__any(grow)) {
            const float m_new = grow ? cm : m_run;
            const float alpha = grow ? sfx_exp2(m_run - cm) : 1.0f;  // (-inf - -inf would be NaN)
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (uint32_t m = 0; m < NM; ++m) O[m] *= alpha;
        }
        const float m_use = m_run == -INFINITY ? 0.0f : m_run;
        float psum = 0.0f;
#pragma unroll
        for (uint32_t e = 0; e < 8; ++e) {
            pf[e] = sfx_exp2(fmaf(pf[e], a.scale_log2, -m_use));
            psum += pf[e];
        }
        l_run += psum;
        // ---- O^T += V^T P^T per 16 dims, P^T scaled by their block's V scales (the
        // product rounded to fp16 once)
        const _Float16* tvs = tb + 32 * D + 32 * NB + gq * 8;
        const _Float16* tv = tb + 32 * D + 64 * NB + lane * 8;
#pragma unroll
        for (uint32_t b = 0; b < NB; ++b) {
            const uint4 vs = *reinterpret_cast<const uint4*>(tvs + 32 * b);
            const half8 pb = __builtin_bit_cast(half8, make_uint4(mul_round2(pf[0], pf[1], vs.x),
                                                                   mul_round2(pf[2], pf[3], vs.y),
                                                                   mul_round2(pf[4], pf[5], vs.z),
                                                                   mul_round2(pf[6], pf[7], vs.w)));
            O[2 * b] = mfma_16x16x32(*reinterpret_cast<const half8*>(tv + 512 * (2 * b)), pb, O[2 * b]);
            O[2 * b + 1] = mfma_16x16x32(*reinterpret_cast<const half8*>(tv + 512 * (2 * b + 1)), pb, O[2 * b + 1]);
        }
        if (s + kExDist < s_end) wait_vmem_le<kPer>();
        else wait_vmem();
        __syncthreads();
    };
    // Steps wholly at or below every row's limit of this wave and inside the split
    // need no mask: key0 + 31 <= wave_lim and key0 + 32 <= key_hi.
    const uint32_t s_plain = max(s_begin, min(s_end, min((wave_lim + 1) / kSufStep, key_hi / kSufStep)));
    for (uint32_t s = s_begin; s < s_plain; ++s) step(s, std::false_type{});
    for (uint32_t s = s_plain; s < s_end; ++s) step(s, std::true_type{});

    // ---- store: PV lane (gq, ci) holds dims 16m + 4gq .. +3 of the wave's row ci
    l_run = rows_reduce(l_run, AddOp{});  // the 4 lanes of a row hold its 32 keys' weights
    const uint32_t orow_i = r0 + wave * 16 + ci;
    if (orow_i >= rows) return;
    const uint32_t ot = orow_i / G;
    const uint32_t oqh = h * G + orow_i % G;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    if (a.splits > 1) {
        // fp32 records (O / l): an fp16 record would round each split's output once more
        const uint32_t rows_cap = a.token_count * G;
        const size_t pr = (static_cast<size_t>(split) * a.g.kv_heads + h) * rows_cap + orow_i;
        float* po = static_cast<float*>(a.part) + pr * D;
#pragma unroll
        for (uint32_t m = 0; m < NM; ++m)
            *reinterpret_cast<float4*>(po + 16 * m + 4 * gq) =
                make_float4(O[m][0] * inv, O[m][1] * inv, O[m][2] * inv, O[m][3] * inv);
        if (gq == 0) {
            float2* ml = reinterpret_cast<float2*>(static_cast<float*>(a.part) +
                                                   part_o_halves(a.splits, a.g.kv_heads, rows_cap, D));
            ml[pr] = make_float2(m_run, l_run);
        }
        return;
    }
    const size_t orow = (static_cast<size_t>(ot) * a.q_heads + oqh) * D;
#pragma unroll
    for (uint32_t m = 0; m < NM; ++m) {
        float4 v;
        v.x = O[m][0] * inv;
        v.y = O[m][1] * inv;
        v.z = O[m][2] * inv;
        v.w = O[m][3] * inv;
        const size_t oi = orow + 16 * m + 4 * gq;
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

// Dims per thread of suffix_combine_kernel.
#ifndef MIIKV_SFX_COMBINE_VEC
#define MIIKV_SFX_COMBINE_VEC 8
#endif
constexpr uint32_t kCombVec = MIIKV_SFX_COMBINE_VEC;

// Merge the splits of each (row, kv head): thread = kCombVec consecutive dims of
// one row.  Token t sees P + t + 1 keys, so splits at or past ceil((P + t + 1) /
// split_keys) hold no key of its row and are skipped; the rest are merged in
// split order (out = sum e^{m_s-M} O_s / sum e^{m_s-M} l_s, 0 when the sum is 0).
template <uint32_t D, typename RecT>
__global__ void __launch_bounds__(256) suffix_combine_kernel(SuffixCombineArgs a) {
    uint32_t T = a.token_count;
    uint32_t P = a.base_position;
    if (a.ps != nullptr) {
        P = a.ps->base_position;
        T = min(T, a.ps->token_count);
    }
    const uint32_t G = a.group;
    const uint32_t h = blockIdx.y;
    const uint32_t idx = blockIdx.x * 256 + threadIdx.x;
    const uint32_t row = idx / (D / kCombVec);
    const uint32_t dv = idx % (D / kCombVec);
    if (row >= T * G) return;
    const uint32_t rows_cap = a.token_count * G;
    const uint32_t t = row / G, g = row % G;
    const uint32_t nsplit = min(a.splits, (P + t + 1 + a.split_keys - 1) / a.split_keys);
    const RecT* po = static_cast<const RecT*>(a.part);
    const float2* ml = reinterpret_cast<const float2*>(po + part_o_halves(a.splits, a.kv_heads, rows_cap, D));
    const size_t oi = (static_cast<size_t>(t) * a.q_heads + h * G + g) * D + kCombVec * dv;
    // Records hold O_s / l_s: each split enters with weight l_s e^{m_s - M}.
    using HalfV = RecT __attribute__((ext_vector_type(kCombVec)));
    float M = -INFINITY, Ls = 0.0f;
    float acc[kCombVec] = {};
    // Batches of kU splits: every load of a batch is issued before the first merge.
    constexpr uint32_t kU = 8;
    float2 e[kU];
    HalfV v[kU];
    auto load_batch = [&](uint32_t sp0) {
#pragma unroll
        for (uint32_t j = 0; j < kU; ++j) {
            const uint32_t sp = min(sp0 + j, nsplit - 1);
            const size_t pr = (static_cast<size_t>(sp) * a.kv_heads + h) * rows_cap + row;
            e[j] = ml[pr];
            v[j] = *reinterpret_cast<const HalfV*>(po + pr * D + kCombVec * dv);
        }
    };
    auto merge_batch = [&](uint32_t sp0) {
#pragma unroll
        for (uint32_t j = 0; j < kU; ++j) {
            const float mn = fmaxf(M, e[j].x);
            if (sp0 + j >= nsplit || mn == -INFINITY) continue;  // past the splits / no key so far
            const float fo = exp2f(M - mn);
            const float ws = e[j].y * exp2f(e[j].x - mn);
            M = mn;
            Ls = Ls * fo + ws;
#pragma unroll
            for (uint32_t c = 0; c < kCombVec; ++c) acc[c] = acc[c] * fo + static_cast<float>(v[j][c]) * ws;
        }
    };
    if (nsplit > 0) load_batch(0);
    // The gate goes out right after the first batch of records: a load in a branch
    // (or still in flight at the head of the batch loop) is waited for before the
    // loads after it are issued, and here everything it waits for is needed next.
    float gv[kCombVec] = {};
    if (a.gate && a.gated_out) {
#pragma unroll
        for (uint32_t c = 0; c < kCombVec; c += 4) {
            const float4 x = *reinterpret_cast<const float4*>(a.gate + oi + c);
            gv[c] = x.x; gv[c + 1] = x.y; gv[c + 2] = x.z; gv[c + 3] = x.w;
        }
    }
    if (nsplit > 0) merge_batch(0);
    for (uint32_t sp0 = kU; sp0 < nsplit; sp0 += kU) {
        load_batch(sp0);
        merge_batch(sp0);
    }
    const float inv = Ls > 0.0f ? 1.0f / Ls : 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < kCombVec; c += 4) {
        const float4 o = make_float4(acc[c] * inv, acc[c + 1] * inv, acc[c + 2] * inv, acc[c + 3] * inv);
        if (a.out) *reinterpret_cast<float4*>(a.out + oi + c) = o;
        if (a.gate && a.gated_out) {
            float4 r;
            r.x = o.x * (1.0f / (1.0f + expf(-gv[c])));
            r.y = o.y * (1.0f / (1.0f + expf(-gv[c + 1])));
            r.z = o.z * (1.0f / (1.0f + expf(-gv[c + 2])));
            r.w = o.w * (1.0f / (1.0f + expf(-gv[c + 3])));
            *reinterpret_cast<float4*>(a.gated_out + oi + c) = r;
        }
    }
}

}  // namespace
}  // namespace miikv

using namespace miikv;

namespace {

// Short suffixes run as a batch of decodes over the one sequence (miikv_decode.hip):
// each decode row set streams the context once for the tokens packed into it (as many
// as fit the MFMA's 16 columns with their query heads), where the MFMA path expands
// the context and runs 32-key steps whose cost barely depends on the token count.
// Measured (graph replays, µs, MFMA path / decodes), 24q/4kv/D256 (2 tokens per row
// set): context 8192 T=1 39.1/12.6, T=4 40.4/21.3, T=8 40.4/25.6, T=16 42.8/36.1;
// context 32768 T=1 78.0/21.8, T=4 79.7/34.1, T=8 80.9/54.8, T=12 82.9/60.1, T=16
// 84.9/82.1.  32q/8kv/D128 (4 per row set): context 32768 T=4 76.0/21.5, T=8
// 76.3/34.2, T=16 76.8/47.0.  Without packing (a device token count), 24q/4kv/D256:
// context 8192 T=12 41.4/36.7, T=16 42.7/46.7; context 32768 T=6 80.3/54.9, T=8
// 80.7/77.8.  So: at most 6 row sets above a 16384-position capacity, 12 at or
// below it.
bool suffix_runs_as_decode(const miikv_view* v, uint32_t q_heads, uint32_t token_count, bool device_count) {
    if (!decode_columns_fit(q_heads / v->kv_heads, v->head_dim)) return false;
    if (token_count > kSuffixDecodeMaxT) return false;
    const uint32_t rows = token_count / suffix_pack(v, q_heads, token_count, device_count);
    return rows <= (view_seq_capacity(v) <= 16384 ? kSuffixDecodeMaxRowsShort : kSuffixDecodeMaxRows);
}

struct SuffixPlan {
    uint32_t splits;
    uint32_t split_keys;
    uint32_t steps;        // expanded steps per kv head
    uint64_t tile_bytes;   // expanded fp16 tiles, all kv heads
    uint64_t part_bytes;   // partial records (splits > 1)
    uint64_t total() const { return tile_bytes + part_bytes; }
};

// Plan for a suffix of `tokens` tokens whose keys end at or before `key_bound`:
// the expanded tiles of every step, and enough splits to fill the chip (at least
// 256 keys per split).  Monotone in key_bound, so a plan made with the cache
// capacity covers any smaller context.
// exact: the plan of suffix_exact_kernel (its tiles and its rows per workgroup).
SuffixPlan make_suffix_plan(const miikv_view* v, uint32_t q_heads, uint32_t tokens, uint64_t key_bound,
                            bool allow_split, uint64_t stride_bound = 0, bool exact = false) {
    SuffixPlan p{1, 0, 0, 0, 0};
    const uint32_t G = q_heads / v->kv_heads;
    const uint32_t rows_per_wg = exact ? kExRows : kSufRows;
    // the tile area holds stride_bound keys per kv head (the capacity for incremental
    // tiles, whose layout must not move between calls), the splits cover key_bound
    p.steps = static_cast<uint32_t>((std::max(key_bound, stride_bound) + kSufStep - 1) / kSufStep);
    p.tile_bytes = static_cast<uint64_t>(v->kv_heads) * p.steps *
                   (exact ? ex_tile_halves(v->head_dim) : tile_halves(v->head_dim)) * 2;
    const uint64_t key_steps = (key_bound + kSufStep - 1) / kSufStep;
    p.split_keys = static_cast<uint32_t>(std::min<uint64_t>(key_steps * kSufStep, 0xffffff00u));
    if (!allow_split) return p;
    const uint64_t wgs = (static_cast<uint64_t>(tokens) * G + rows_per_wg - 1) / rows_per_wg * v->kv_heads;
    // Splits: as many as keep every workgroup resident in one round (the
    // per-workgroup cost does not shrink with more concurrent workgroups, so a
    // second partial round costs a full one), at least 256 keys each.
    const uint64_t by_keys = std::min<uint64_t>((key_bound + 255) / 256, kSufMaxSplits);
    uint64_t want = std::max<uint64_t>(1, kSufSlots / wgs);
    want = std::max<uint64_t>(1, std::min<uint64_t>({want, by_keys, kSufMaxSplits}));
    if (want <= 1) return p;
    const uint64_t unit = kSufStep;
    const uint64_t cpw = (key_bound + want * unit - 1) / (want * unit);
    const uint32_t split_keys = static_cast<uint32_t>(cpw * unit);
    const uint32_t splits = static_cast<uint32_t>((key_bound + split_keys - 1) / split_keys);
    if (splits <= 1) return p;
    p.splits = splits;
    p.split_keys = split_keys;
    // Records sized for `want` (>= splits): a plan for a shorter context never needs more.
    p.part_bytes = want * v->kv_heads * tokens * G * (exact ? 4 * v->head_dim + 8 : part_row_bytes(v->head_dim));
    return p;
}

}  // namespace

// Workspace of miikv_suffix_attn: the expanded fp16 tiles of the context and,
// for split-K, the partial records; planned for the cache capacity, so it serves
// any base position (and a device prefill state).
extern "C" uint64_t miikv_suffix_workspace_bytes(const miikv_view* view, uint32_t q_heads, uint32_t token_count) {
    if (validate_view(view) != MIIKV_OK || q_heads == 0 || q_heads % view->kv_heads != 0 || token_count == 0)
        return 0;
    // Room for either path and for incremental tiles: the tiles of every key of the
    // capacity, then the larger of the split records and a short suffix's decode
    // records (a short suffix keeping the tiles current needs both).
    const uint64_t cap = view_seq_capacity(view);
    uint64_t dec = 0;
    if (suffix_runs_as_decode(view, q_heads, token_count, false) ||
        suffix_runs_as_decode(view, q_heads, token_count, true))
        dec = suffix_by_decode_bytes(view, q_heads, token_count, static_cast<uint32_t>(std::min<uint64_t>(cap, 0xffffffffu)));
    const SuffixPlan p = make_suffix_plan(view, q_heads, token_count, cap, true);
    return p.tile_bytes + std::max(dec, p.part_bytes);
}

// Exact route: the tiles (kept for MIIKV_SUFFIX_TILES_CURRENT, whose decode-route
// records sit above them) plus the records of every token as a decode.
extern "C" uint64_t miikv_suffix_workspace_bytes_ex(const miikv_view* view, uint32_t q_heads, uint32_t token_count,
                                                    uint32_t flags) {
    if ((flags & ~(MIIKV_SUFFIX_TILES_CURRENT | MIIKV_SUFFIX_EXACT)) != 0) return 0;
    const uint64_t base = miikv_suffix_workspace_bytes(view, q_heads, token_count);
    if (base == 0 || (flags & MIIKV_SUFFIX_EXACT) == 0) return base;
    if (!decode_columns_fit(q_heads / view->kv_heads, view->head_dim)) return 0;
    const uint64_t cap = view_seq_capacity(view);
    const SuffixPlan tiles = make_suffix_plan(view, q_heads, token_count, cap, false);
    const uint32_t cap32 = static_cast<uint32_t>(std::min<uint64_t>(cap, 0xffffffffu));
    const SuffixPlan xp = make_suffix_plan(view, q_heads, token_count, cap, true, 0, true);
    return std::max({base, tiles.tile_bytes + suffix_by_decode_bytes(view, q_heads, token_count, cap32),
                     xp.total()});
}

// The split merge of the MFMA kernels (the records of either kernel have one layout).
// f32: the exact kernel's fp32 records.
static void launch_suffix_combine(const miikv_view* view, uint32_t q_heads, uint32_t G, uint32_t token_count,
                                  uint32_t base_position, const miikv_prefill_state* prefill_state,
                                  const SuffixPlan& plan, void* part, float* out, const float* gate, float* gated_out,
                                  hipStream_t s, bool f32 = false) {
    SuffixCombineArgs c{};
    c.kv_heads = view->kv_heads;
    c.q_heads = q_heads;
    c.group = G;
    c.token_count = token_count;
    c.base_position = base_position;
    c.ps = prefill_state;
    c.split_keys = plan.split_keys;
    c.splits = plan.splits;
    c.part = part;
    c.out = out;
    c.gate = gate;
    c.gated_out = gated_out;
    const uint64_t threads = static_cast<uint64_t>(token_count) * G * (view->head_dim / kCombVec);
    const dim3 cgrid(static_cast<uint32_t>((threads + 255) / 256), view->kv_heads);
    if (view->head_dim == 128) {
        if (f32) hipLaunchKernelGGL((suffix_combine_kernel<128, float>), cgrid, dim3(256), 0, s, c);
        else hipLaunchKernelGGL((suffix_combine_kernel<128, _Float16>), cgrid, dim3(256), 0, s, c);
    } else {
        if (f32) hipLaunchKernelGGL((suffix_combine_kernel<256, float>), cgrid, dim3(256), 0, s, c);
        else hipLaunchKernelGGL((suffix_combine_kernel<256, _Float16>), cgrid, dim3(256), 0, s, c);
    }
}

static miikv_status suffix_impl(const miikv_view* view, const uint16_t* k_new, const uint16_t* v_new, const void* q,
                                uint32_t q_dtype, uint32_t q_heads, float scale, uint32_t token_count,
                                uint32_t base_position, uint32_t seq, const miikv_prefill_state* prefill_state,
                                uint32_t flags, float* out, const float* gate, float* gated_out, void* workspace,
                                uint64_t workspace_bytes, void* stream) {
    const int st = validate_view(view);
    if (st != MIIKV_OK) return st;
    if (q == nullptr || q_heads == 0 || q_heads % view->kv_heads != 0 || !std::isfinite(scale)) return MIIKV_EINVAL;
    if (q_dtype != MIIKV_DTYPE_F16 && q_dtype != MIIKV_DTYPE_F32) return MIIKV_EINVAL;
    const uint32_t G = q_heads / view->kv_heads;
    if (out == nullptr && !(gate != nullptr && gated_out != nullptr)) return MIIKV_EINVAL;
    if ((gate == nullptr) != (gated_out == nullptr)) return MIIKV_EINVAL;
    if (view->layout == MIIKV_LAYOUT_CONTIGUOUS && seq != 0) return MIIKV_EINVAL;
    if ((flags & ~(MIIKV_SUFFIX_TILES_CURRENT | MIIKV_SUFFIX_EXACT)) != 0) return MIIKV_EINVAL;
    const bool current = (flags & MIIKV_SUFFIX_TILES_CURRENT) != 0;
    const bool exact = (flags & MIIKV_SUFFIX_EXACT) != 0;
    if (exact && !decode_columns_fit(G, view->head_dim)) return MIIKV_EUNSUPPORTED;
    if (token_count == 0) return MIIKV_OK;
    if (k_new != nullptr && view->quant_mode != MIIKV_KV_Q8_Q8) return MIIKV_EUNSUPPORTED;  // stores q8 rows
    const uint64_t cap = view_seq_capacity(view);
    if (prefill_state == nullptr && static_cast<uint64_t>(base_position) + token_count > cap) return MIIKV_EINVAL;
    const uint64_t rows = static_cast<uint64_t>(token_count) * G;
    const uint64_t blocks = (rows + kSufRows - 1) / kSufRows;
    if (blocks > 0x7fffffffu || static_cast<uint64_t>(token_count) * view->kv_heads > 0x7fffffffu)
        return MIIKV_EINVAL;
    // The key bound: the known context (host base position) or the capacity (device
    // state).  A workspace of miikv_suffix_workspace_bytes() bytes always suffices;
    // one holding just the tiles runs a single split.
    const uint64_t bound = prefill_state ? cap : static_cast<uint64_t>(base_position) + token_count;
    if (workspace == nullptr) return MIIKV_EWORKSPACE;
    const uint32_t bound32 = static_cast<uint32_t>(std::min<uint64_t>(bound, 0xffffffffu));
    hipStream_t s = static_cast<hipStream_t>(stream);
    _Float16* tiles = static_cast<_Float16*>(workspace);
    // Incremental tiles: the tile area holds every key of the capacity at a fixed
    // stride; steps below the base position are current, the rest are expanded here.
    const uint64_t stride_bound = current ? cap : 0;
    const uint32_t host_step0 = current && prefill_state == nullptr ? base_position / kSufStep : 0u;
    auto expand = [&](const SuffixPlan& plan, bool append) {
        ExpandArgs e{};
        e.g = make_geo(*view);
        e.seq = seq;
        e.key_count = bound32;
        e.ps = prefill_state;
        e.steps = plan.steps;
        e.tiles = tiles;
        e.k_new = append ? k_new : nullptr;
        e.v_new = append ? v_new : nullptr;
        e.token_count = token_count;
        e.base_position = base_position;
        e.step0 = host_step0;
        e.current = current ? 1u : 0u;
        const uint32_t key_steps = static_cast<uint32_t>((bound + kSufStep - 1) / kSufStep);
        const dim3 egrid(key_steps - host_step0, view->kv_heads);
        if (append) {
            if (view->head_dim == 128) hipLaunchKernelGGL((expand_kernel<128, true>), egrid, dim3(256), 0, s, e);
            else hipLaunchKernelGGL((expand_kernel<256, true>), egrid, dim3(256), 0, s, e);
        } else {
            if (view->head_dim == 128) hipLaunchKernelGGL((expand_kernel<128, false>), egrid, dim3(256), 0, s, e);
            else hipLaunchKernelGGL((expand_kernel<256, false>), egrid, dim3(256), 0, s, e);
        }
    };
    // (a workspace sized for the MFMA path alone runs that path)
    const SuffixPlan tile_plan = make_suffix_plan(view, q_heads, token_count, bound, false, stride_bound);
    const uint64_t dec_off = current ? tile_plan.tile_bytes : 0;  // the tiles stay below the records
    const bool short_suffix = suffix_runs_as_decode(view, q_heads, token_count, prefill_state != nullptr);
    // MIIKV_SUFFIX_EXACT: a long suffix over q8 planes runs the exact-product MFMA
    // kernels; short suffixes, other quant modes and chunked prefill (whose tiles keep
    // the plain layout) run every token as a decode.
    const bool exact_mfma = exact && !current && !short_suffix && view->quant_mode == MIIKV_KV_Q8_Q8;
    if (exact_mfma) {
        if (k_new != nullptr) {  // the suffix's own rows first, with the append rule
            const miikv_status ast = miikv_append_f16(view, k_new, v_new, token_count, base_position, seq,
                                                      prefill_state, nullptr, stream);
            if (ast != MIIKV_OK) return ast;
        }
        SuffixPlan xp = make_suffix_plan(view, q_heads, token_count, bound, true, 0, true);
        if (workspace_bytes < xp.total()) {
            xp = make_suffix_plan(view, q_heads, token_count, bound, false, 0, true);
            if (workspace_bytes < xp.total()) return MIIKV_EWORKSPACE;
        }
        if (xp.steps > 65535u * 64u) return MIIKV_EINVAL;
        const uint64_t xblocks = (rows + kExRows - 1) / kExRows;
        ExpandArgs e{};
        e.g = make_geo(*view);
        e.seq = seq;
        e.key_count = bound32;
        e.ps = prefill_state;
        e.steps = xp.steps;
        e.tiles = tiles;
        e.k_new = nullptr;
        e.v_new = nullptr;
        e.token_count = token_count;
        e.base_position = base_position;
        e.step0 = 0;
        e.current = 0;
        const dim3 egrid(static_cast<uint32_t>((bound + kSufStep - 1) / kSufStep), view->kv_heads);
        if (view->head_dim == 128) hipLaunchKernelGGL((expand_exact_kernel<128>), egrid, dim3(256), 0, s, e);
        else hipLaunchKernelGGL((expand_exact_kernel<256>), egrid, dim3(256), 0, s, e);
        SuffixArgs a{};
        a.g = make_geo(*view);
        a.q = q;
        a.q_f32 = q_dtype == MIIKV_DTYPE_F32;
        a.q_heads = q_heads;
        a.group = G;
        a.scale_log2 = scale * kLog2eS;
        a.token_count = token_count;
        a.base_position = base_position;
        a.ps = prefill_state;
        a.split_keys = xp.split_keys;
        a.splits = xp.splits;
        a.row_blocks = static_cast<uint32_t>(xblocks);
        a.steps = xp.steps;
        a.tiles = tiles;
        a.part = static_cast<uint8_t*>(workspace) + xp.tile_bytes;
        a.out = out;
        a.gate = gate;
        a.gated_out = gated_out;
        const uint64_t xwgs = (static_cast<uint64_t>(view->kv_heads) * xp.splits * xblocks + 7) / 8 * 8;
        if (xwgs > 0x7fffffffu) return MIIKV_EINVAL;
        const dim3 xgrid(static_cast<uint32_t>(xwgs)), xblock(64 * kExWaves);
        if (view->head_dim == 128) {
            if (a.q_f32) hipLaunchKernelGGL((suffix_exact_kernel<128, true>), xgrid, xblock, 0, s, a);
            else hipLaunchKernelGGL((suffix_exact_kernel<128, false>), xgrid, xblock, 0, s, a);
        } else {
            if (a.q_f32) hipLaunchKernelGGL((suffix_exact_kernel<256, true>), xgrid, xblock, 0, s, a);
            else hipLaunchKernelGGL((suffix_exact_kernel<256, false>), xgrid, xblock, 0, s, a);
        }
        if (xp.splits > 1) launch_suffix_combine(view, q_heads, G, token_count, base_position, prefill_state, xp,
                                                 a.part, out, gate, gated_out, s, true);
        return hip_status(hipGetLastError());
    }
    const bool by_decode = exact || short_suffix;
    const bool dec_fits = workspace_bytes >= dec_off + suffix_by_decode_bytes(view, q_heads, token_count, bound32);
    if (exact && !dec_fits) return MIIKV_EWORKSPACE;
    if (by_decode && dec_fits) {
        // the suffix's own rows first; every token then reads its context from the cache
        if (k_new != nullptr) {
            const miikv_status ast = miikv_append_f16(view, k_new, v_new, token_count, base_position, seq,
                                                      prefill_state, nullptr, stream);
            if (ast != MIIKV_OK) return ast;
        }
        if (current) {
            if (tile_plan.steps > 65535u * 64u) return MIIKV_EINVAL;
            expand(tile_plan, false);  // the suffix's own steps, for the next call
        }
        return suffix_by_decode(view, q, q_dtype, q_heads, scale, token_count, base_position, seq, prefill_state,
                                bound32, out, gate, gated_out, static_cast<uint8_t*>(workspace) + dec_off,
                                workspace_bytes - dec_off, stream);
    }
    SuffixPlan plan = make_suffix_plan(view, q_heads, token_count, bound, true, stride_bound);
    if (workspace_bytes < plan.total()) {
        plan = tile_plan;
        if (workspace_bytes < plan.total()) return MIIKV_EWORKSPACE;
    }
    if (plan.steps > 65535u * 64u) return MIIKV_EINVAL;

    expand(plan, k_new != nullptr);

    SuffixArgs a{};
    a.g = make_geo(*view);
    a.q = q;
    a.q_f32 = q_dtype == MIIKV_DTYPE_F32;
    a.q_heads = q_heads;
    a.group = G;
    a.scale_log2 = scale * kLog2eS;
    a.token_count = token_count;
    a.base_position = base_position;
    a.ps = prefill_state;
    a.split_keys = plan.split_keys;
    a.splits = plan.splits;
    a.row_blocks = static_cast<uint32_t>(blocks);
    a.steps = plan.steps;
    a.tiles = tiles;
    a.part = static_cast<uint8_t*>(workspace) + plan.tile_bytes;
    a.out = out;
    a.gate = gate;
    a.gated_out = gated_out;
    // Short splits: the splits of a row block on one XCD (config 4, 55 steps per
    // split: 135.0 -> 131.7 us; the ladder at P = 4096 3.5% faster); long ones keep
    // the (kv head, split)-major order, whose tiles more row blocks share (P = 65536:
    // 0.3% slower the other way, P = 32768 level).
    a.rows_together = plan.splits > 1 && plan.split_keys <= 128 * kSufStep ? 1u : 0u;
    const uint64_t groups = static_cast<uint64_t>(view->kv_heads) * plan.splits;
    const uint64_t wgs = (groups * blocks + 7) / 8 * 8;
    if (wgs > 0x7fffffffu) return MIIKV_EINVAL;
    const dim3 grid(static_cast<uint32_t>(wgs));
    if (view->head_dim == 128) hipLaunchKernelGGL(suffix_kernel<128>, grid, dim3(64 * kSufWaves), 0, s, a);
    else hipLaunchKernelGGL(suffix_kernel<256>, grid, dim3(64 * kSufWaves), 0, s, a);
    if (plan.splits > 1) launch_suffix_combine(view, q_heads, G, token_count, base_position, prefill_state, plan,
                                               a.part, out, gate, gated_out, s);
    return hip_status(hipGetLastError());
}

extern "C" miikv_status miikv_suffix_attn(const miikv_view* view, const void* q, uint32_t q_dtype, uint32_t q_heads,
                                          float scale, uint32_t token_count, uint32_t base_position, uint32_t seq,
                                          const miikv_prefill_state* prefill_state, float* out, const float* gate,
                                          float* gated_out, void* workspace, uint64_t workspace_bytes,
                                          void* stream) {
    return suffix_impl(view, nullptr, nullptr, q, q_dtype, q_heads, scale, token_count, base_position, seq,
                       prefill_state, 0u, out, gate, gated_out, workspace, workspace_bytes, stream);
}

extern "C" miikv_status miikv_suffix_append_attn(const miikv_view* view, const uint16_t* k_new, const uint16_t* v_new,
                                                 const void* q, uint32_t q_dtype, uint32_t q_heads, float scale,
                                                 uint32_t token_count, uint32_t base_position, uint32_t seq,
                                                 const miikv_prefill_state* prefill_state, float* out,
                                                 const float* gate, float* gated_out, void* workspace,
                                                 uint64_t workspace_bytes, void* stream) {
    if (k_new == nullptr || v_new == nullptr) return MIIKV_EINVAL;
    return suffix_impl(view, k_new, v_new, q, q_dtype, q_heads, scale, token_count, base_position, seq,
                       prefill_state, 0u, out, gate, gated_out, workspace, workspace_bytes, stream);
}

extern "C" miikv_status miikv_suffix_attn_ex(const miikv_view* view, const uint16_t* k_new, const uint16_t* v_new,
                                             const void* q, uint32_t q_dtype, uint32_t q_heads, float scale,
                                             uint32_t token_count, uint32_t base_position, uint32_t seq,
                                             const miikv_prefill_state* prefill_state, uint32_t flags, float* out,
                                             const float* gate, float* gated_out, void* workspace,
                                             uint64_t workspace_bytes, void* stream) {
    if ((k_new == nullptr) != (v_new == nullptr)) return MIIKV_EINVAL;
    return suffix_impl(view, k_new, v_new, q, q_dtype, q_heads, scale, token_count, base_position, seq,
                       prefill_state, flags, out, gate, gated_out, workspace, workspace_bytes, stream);
}
