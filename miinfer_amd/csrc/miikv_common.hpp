// Shared device helpers for the miikv kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>

#include "miikv.h"
#include "miikv_rope.h"

namespace miikv {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr uint32_t kWave = 64;
constexpr uint32_t kChunk = 32;   // tokens per wave step (one V group, two K tiles)
constexpr uint32_t kTile = 16;    // tokens per K tile (MFMA M/N)

// Geometry of a cache view, passed by value to kernels.
struct Geo {
    int8_t* k_codes;
    uint16_t* k_scales;
    int8_t* v_codes;
    uint16_t* v_scales;
    const int32_t* table;
    uint32_t layout;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t page_tokens;
    uint32_t table_stride;
    uint32_t num_pages;
    // fp16 planes (quant modes FP16_*): the plane holds the fp16 rows in the same
    // tiled element order as the codes, 2 bytes per element, and has no scales.
    uint32_t k_f16;
    uint32_t v_f16;
};

inline bool mode_k_f16(uint32_t mode) { return mode == MIIKV_KV_FP16_FP16 || mode == MIIKV_KV_FP16_Q8; }
inline bool mode_v_f16(uint32_t mode) { return mode == MIIKV_KV_FP16_FP16 || mode == MIIKV_KV_Q8_FP16; }

inline Geo make_geo(const miikv_view& v) {
    Geo g;
    g.k_codes = v.k_codes;
    g.k_scales = v.k_scales;
    g.v_codes = v.v_codes;
    g.v_scales = v.v_scales;
    g.table = v.block_table;
    g.layout = v.layout;
    g.kv_heads = v.kv_heads;
    g.head_dim = v.head_dim;
    g.page_tokens = v.page_tokens;
    g.table_stride = v.table_stride;
    g.num_pages = v.num_pages;
    g.k_f16 = mode_k_f16(v.quant_mode) ? 1u : 0u;
    g.v_f16 = mode_v_f16(v.quant_mode) ? 1u : 0u;
    return g;
}

// Slab index (page * kv_heads + head) holding token `pos` of sequence `seq`.
__device__ __forceinline__ size_t slab_of(const Geo& g, uint32_t seq, uint32_t pos, uint32_t head) {
    uint32_t page = 0;
    if (g.layout == MIIKV_LAYOUT_PAGED) {
        page = static_cast<uint32_t>(g.table[static_cast<size_t>(seq) * g.table_stride + pos / g.page_tokens]);
    }
    return static_cast<size_t>(page) * g.kv_heads + head;
}

// As slab_of, with the page index clamped into [0, num_pages): for speculative
// loads whose table entry may not be set yet (the data is discarded).
__device__ __forceinline__ size_t slab_of_clamped(const Geo& g, uint32_t seq, uint32_t pos, uint32_t head) {
    uint32_t page = 0;
    if (g.layout == MIIKV_LAYOUT_PAGED) {
        page = static_cast<uint32_t>(g.table[static_cast<size_t>(seq) * g.table_stride + pos / g.page_tokens]);
        page = min(page, g.num_pages - 1);
    }
    return static_cast<size_t>(page) * g.kv_heads + head;
}

// Byte offset of (token tp within the slab, dim d) in a K-code slab.
__device__ __forceinline__ uint32_t k_code_offset(uint32_t tp, uint32_t d, uint32_t D) {
    const uint32_t T = tp >> 4, m = tp & 15;
    const uint32_t c = d >> 6, e = (d >> 5) & 1, gq = (d >> 3) & 3, j = d & 7;
    return T * (16 * D) + c * 1024 + gq * 256 + m * 16 + e * 8 + j;
}

// Byte offset of (token tp within the slab, dim d) in a V-code slab: 32-token
// groups, token-contiguous per dim, tokens ordered (G, J, I) for t = 16J + 4G + I.
__device__ __forceinline__ uint32_t v_code_offset(uint32_t tp, uint32_t d, uint32_t D) {
    const uint32_t H = tp >> 5, J = (tp >> 4) & 1, G = (tp >> 2) & 3, I = tp & 3;
    return H * (32 * D) + d * 32 + G * 8 + J * 4 + I;
}

// Butterfly reductions over aligned lane groups of 2..64 lanes without an LDS
// round trip: DPP quad permutes for partners 1 and 2, the row half-mirror and
// mirror for partners in the other quad / half-row (within a group whose lanes
// already agree these pair the same groups as xor 4 and xor 8), and the gfx950
// permlane swaps for partners 16 and 32 lanes away. Every lane of a group ends
// with the same value, combined in the same tree as the xor-shuffle butterfly.
template <typename T>
__device__ __forceinline__ T lane_bits_to(int v) { return __builtin_bit_cast(T, v); }
template <uint32_t kCtrl, typename T>
__device__ __forceinline__ T dpp_mov(T x) {
    return lane_bits_to<T>(__builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xF, 0xF, false));
}
// The swap results are copied out element by element before any bit cast: clang
// lowers __builtin_bit_cast of an element of the returned vector to element 0.
template <typename T, typename Op>
__device__ __forceinline__ T swap16_reduce(T x, Op op) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return op(__builtin_bit_cast(T, r0), __builtin_bit_cast(T, r1));
}
template <typename T, typename Op>
__device__ __forceinline__ T swap32_reduce(T x, Op op) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return op(__builtin_bit_cast(T, r0), __builtin_bit_cast(T, r1));
}
// Reduce over the kLanes-lane group (lanes [k*kLanes, (k+1)*kLanes)) holding x.
template <uint32_t kLanes, typename T, typename Op>
__device__ __forceinline__ T group_reduce(T x, Op op) {
    static_assert(kLanes >= 2 && kLanes <= 64 && (kLanes & (kLanes - 1)) == 0, "power of two");
    x = op(x, dpp_mov<0xB1>(x));                        // quad_perm [1,0,3,2]
    if constexpr (kLanes >= 4) x = op(x, dpp_mov<0x4E>(x));   // quad_perm [2,3,0,1]
    if constexpr (kLanes >= 8) x = op(x, dpp_mov<0x141>(x));  // row_half_mirror
    if constexpr (kLanes >= 16) x = op(x, dpp_mov<0x140>(x)); // row_mirror
    if constexpr (kLanes >= 32) x = swap16_reduce(x, op);
    if constexpr (kLanes >= 64) x = swap32_reduce(x, op);
    return x;
}
struct MaxOp {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct AddOp {
    template <typename T>
    __device__ T operator()(T a, T b) const { return a + b; }
};
// Reduce across the four 16-lane rows (partners 16 and 32 lanes away) only.
template <typename T, typename Op>
__device__ __forceinline__ T rows_reduce(T x, Op op) {
    return swap32_reduce(swap16_reduce(x, op), op);
}

// q8_0 quantization of 16 values held by this lane; its partner lane (lane ^ 1)
// holds the other 16 values of the same 32-value block.  Rule of
// gfx906/kernels/qwen3_primitives.hip:7285-7322 applied per block.
__device__ __forceinline__ void quantize16(const float (&x)[16], int8_t (&q)[16], float& scale_out) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(x[i]));
    amax = group_reduce<2>(amax, MaxOp{});
    const float scale = (amax > 0.0f) ? (amax / 127.0f) : 1.0f;
    const float inv = (scale > 0.0f) ? (1.0f / scale) : 1.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int r = __float2int_rn(x[i] * inv);
        r = max(-128, min(127, r));
        q[i] = static_cast<int8_t>(r);
    }
    scale_out = scale;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
    __half h = __float2half_rn(x);
    return __half_as_ushort(h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return __half2float(__ushort_as_half(b));
}

// 16 consecutive fp16 values (two 16-byte words) -> fp32.
__device__ __forceinline__ void unpack16_f16(const uint4 (&r)[2], float (&x)[16]) {
    const uint32_t w[8] = {r[0].x, r[0].y, r[0].z, r[0].w, r[1].x, r[1].y, r[1].z, r[1].w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        x[2 * i] = f16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
        x[2 * i + 1] = f16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
}
__device__ __forceinline__ void load16_f16(const uint16_t* p, float (&x)[16]) {
    const uint4 r[2] = {*reinterpret_cast<const uint4*>(p), *reinterpret_cast<const uint4*>(p + 8)};
    unpack16_f16(r, x);
}

// Four signed int8 codes (one dword) -> four exact fp16 values, two per dword.
// u = c ^ 0x80 = c + 128; the fp16 with bits 0x6400|u equals 1024 + u, so
// subtracting 1152 yields c exactly.
__device__ __forceinline__ void codes4_to_half(uint32_t w, half2v& lo, half2v& hi) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = __builtin_bit_cast(half2v, a) - bias;
    hi = __builtin_bit_cast(half2v, b) - bias;
}

// Eight codes (two dwords) -> half8 in code order.
__device__ __forceinline__ half8 codes8_to_half8(uint32_t w0, uint32_t w1) {
    half2v a, b, c, d;
    codes4_to_half(w0, a, b);
    codes4_to_half(w1, c, d);
    half8 r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
    return r;
}

// Four codes (one dword) -> half4 in code order.
__device__ __forceinline__ half4 codes4_to_half4(uint32_t w) {
    half2v a, b;
    codes4_to_half(w, a, b);
    half4 r;
    r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
    return r;
}

// Biased variants: four codes -> fp16 (code + 1152), exact, without the subtraction.
// Callers remove 1152 * (sum of the other operand) themselves.
__device__ __forceinline__ half4 codes4_to_half4_biased(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    return __builtin_bit_cast(half4, make_uint2(a, b));
}

__device__ __forceinline__ half8 codes8_to_half8_biased(uint32_t w0, uint32_t w1) {
    const uint32_t u0 = w0 ^ 0x80808080u;
    const uint32_t u1 = w1 ^ 0x80808080u;
    const uint4 r = make_uint4(__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u),
                               __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u),
                               __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u),
                               __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u));
    return __builtin_bit_cast(half8, r);
}

__device__ __forceinline__ float4v mfma_16x16x32(half8 a, half8 b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float4v mfma_16x16x16(half4 a, half4 b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

inline int hip_status(hipError_t e) { return e == hipSuccess ? MIIKV_OK : -static_cast<int>(e); }

}  // namespace miikv
