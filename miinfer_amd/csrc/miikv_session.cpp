// Persistent session files (.miinfer): the reference's on-disk prefix state
// (include/miinfer/prefill_v2/persistent_session.hpp:18-69,
// src/prefill_v2/persistent_session.cpp:27-320) for caches of every quant mode in
// any layout.  Host code over the HIP runtime: the KV bytes move through
// miikv_export_canonical / miikv_import_canonical and one device staging buffer.
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <ctime>
#include <filesystem>
#include <fstream>
#include <string>
#include <vector>

#include "miikv.h"

static_assert(sizeof(miikv_session_header) == 157, "packed header layout of persistent_session.hpp:18-34");

namespace {

constexpr char kMagic[4] = {'M', 'I', 'S', 'S'};

struct Geometry {
    uint32_t kv_heads = 0, head_dim = 0, quant_mode = 0;
    bool k_f16 = false, v_f16 = false;
    uint64_t k_head = 0, v_head = 0;  // raw bytes of one head's K (V) part: rows, then scales
    uint64_t layer_bytes = 0;         // kv_heads * (k_head + v_head)
};

uint64_t view_capacity(const miikv_view& v) {
    return v.layout == MIIKV_LAYOUT_PAGED ? static_cast<uint64_t>(v.table_stride) * v.page_tokens
                                          : static_cast<uint64_t>(v.page_tokens);
}

bool is_f16_k(uint32_t mode) { return mode == MIIKV_KV_FP16_FP16 || mode == MIIKV_KV_FP16_Q8; }
bool is_f16_v(uint32_t mode) { return mode == MIIKV_KV_FP16_FP16 || mode == MIIKV_KV_Q8_FP16; }

}  // namespace

// Session-file kv_quant_mode of a view quant mode, and back (0xff: none).
extern "C" uint32_t miikv_session_kv_mode(uint32_t view_quant_mode) {
    switch (view_quant_mode) {
        case MIIKV_KV_FP16_FP16: return MIIKV_SESSION_KV_FP16_FP16;
        case MIIKV_KV_Q8_FP16: return MIIKV_SESSION_KV_Q8_0_32_FP16;
        case MIIKV_KV_FP16_Q8: return MIIKV_SESSION_KV_FP16_Q8_0_32;
        case MIIKV_KV_Q8_Q8: return MIIKV_SESSION_KV_Q8_0_32;
        default: return 0xffu;
    }
}

namespace {

// Every layer must share one geometry and quant mode (the file splits kv_bytes
// evenly, persistent_session.cpp:251) and hold P tokens.
bool layers_geometry(const miikv_view* layers, uint32_t count, uint32_t P, Geometry& g) {
    if (layers == nullptr || count == 0) return false;
    for (uint32_t i = 0; i < count; ++i) {
        const miikv_view& v = layers[i];
        if (miikv_session_kv_mode(v.quant_mode) == 0xffu || v.head_dim == 0 || v.head_dim % 32 != 0 ||
            v.kv_heads == 0)
            return false;
        if (i == 0) {
            g.kv_heads = v.kv_heads;
            g.head_dim = v.head_dim;
            g.quant_mode = v.quant_mode;
        } else if (v.kv_heads != g.kv_heads || v.head_dim != g.head_dim || v.quant_mode != g.quant_mode) {
            return false;
        }
        if (P > view_capacity(v)) return false;
    }
    g.k_f16 = is_f16_k(g.quant_mode);
    g.v_f16 = is_f16_v(g.quant_mode);
    const uint64_t rows16 = 2ull * P * g.head_dim;                       // fp16 rows
    const uint64_t rows8 = static_cast<uint64_t>(P) * g.head_dim + 2ull * P * (g.head_dim / 32);  // codes + scales
    g.k_head = g.k_f16 ? rows16 : rows8;
    g.v_head = g.v_f16 ? rows16 : rows8;
    g.layer_bytes = static_cast<uint64_t>(g.kv_heads) * (g.k_head + g.v_head);
    return true;
}

uint64_t sum_bytes(const uint64_t* bytes, uint32_t n) {
    uint64_t t = 0;
    for (uint32_t i = 0; i < n; ++i) t += bytes[i];
    return t;
}

std::string field(const char* s, size_t cap) { return std::string(s, strnlen(s, cap)); }

// Device staging for one layer: canonical K codes, K scales, V codes, V scales.
struct Staging {
    int8_t* kc = nullptr;
    uint16_t* ks = nullptr;
    int8_t* vc = nullptr;
    uint16_t* vs = nullptr;
    void* base = nullptr;
    ~Staging() {
        if (base) (void)hipFree(base);
    }
    hipError_t alloc(uint32_t P, const Geometry& g) {
        // an fp16 plane's rows take 2 bytes per element in the codes buffer
        const size_t elems = static_cast<size_t>(P) * g.kv_heads * g.head_dim;
        const size_t scales = static_cast<size_t>(P) * g.kv_heads * (g.head_dim / 32) * 2;
        const size_t kc_al = (elems * (g.k_f16 ? 2 : 1) + 255) / 256 * 256;
        const size_t vc_al = (elems * (g.v_f16 ? 2 : 1) + 255) / 256 * 256;
        const size_t s_al = (scales + 255) / 256 * 256;
        hipError_t e = hipMalloc(&base, kc_al + vc_al + 2 * s_al);
        if (e != hipSuccess) return e;
        uint8_t* p = static_cast<uint8_t*>(base);
        kc = reinterpret_cast<int8_t*>(p);
        ks = g.k_f16 ? nullptr : reinterpret_cast<uint16_t*>(p + kc_al);
        vc = reinterpret_cast<int8_t*>(p + kc_al + s_al);
        vs = g.v_f16 ? nullptr : reinterpret_cast<uint16_t*>(p + kc_al + s_al + vc_al);
        return hipSuccess;
    }
};

// Raw layout of one layer (kv_cache.cpp:227-297): for each kv head its K rows (fp16
// [P][D], or q8 codes [P][D] then scales [P][D/32]), then the same for V.  Host offsets
// of head h's parts and their device spans in the staging buffer.
struct RawPlanes {
    uint64_t k_rows, k_scales, v_rows, v_scales;  // file offsets
    uint64_t k_row_bytes, v_row_bytes, scale_bytes;  // per head
};
RawPlanes raw_planes(uint32_t P, const Geometry& g, uint32_t h) {
    RawPlanes r;
    r.k_row_bytes = static_cast<uint64_t>(P) * g.head_dim * (g.k_f16 ? 2 : 1);
    r.v_row_bytes = static_cast<uint64_t>(P) * g.head_dim * (g.v_f16 ? 2 : 1);
    r.scale_bytes = 2ull * P * (g.head_dim / 32);
    const uint64_t v0 = g.k_head * g.kv_heads;
    r.k_rows = g.k_head * h;
    r.k_scales = r.k_rows + r.k_row_bytes;
    r.v_rows = v0 + g.v_head * h;
    r.v_scales = r.v_rows + r.v_row_bytes;
    return r;
}

// One layer between the staging buffer and its raw bytes: device -> host (save) or
// host -> device (load), for every head.
hipError_t move_layer(const Staging& st, const Geometry& g, uint32_t P, uint8_t* raw, bool to_host, hipStream_t s) {
    for (uint32_t hd = 0; hd < g.kv_heads; ++hd) {
        const RawPlanes rp = raw_planes(P, g, hd);
        struct Part {
            uint8_t* dev;
            uint64_t off, bytes;
        } parts[4] = {
            {reinterpret_cast<uint8_t*>(st.kc) + hd * rp.k_row_bytes, rp.k_rows, rp.k_row_bytes},
            {g.k_f16 ? nullptr : reinterpret_cast<uint8_t*>(st.ks) + hd * rp.scale_bytes, rp.k_scales,
             g.k_f16 ? 0 : rp.scale_bytes},
            {reinterpret_cast<uint8_t*>(st.vc) + hd * rp.v_row_bytes, rp.v_rows, rp.v_row_bytes},
            {g.v_f16 ? nullptr : reinterpret_cast<uint8_t*>(st.vs) + hd * rp.scale_bytes, rp.v_scales,
             g.v_f16 ? 0 : rp.scale_bytes},
        };
        for (const Part& pt : parts) {
            if (pt.bytes == 0) continue;
            const hipError_t e = to_host ? hipMemcpyAsync(raw + pt.off, pt.dev, pt.bytes, hipMemcpyDeviceToHost, s)
                                         : hipMemcpyAsync(pt.dev, raw + pt.off, pt.bytes, hipMemcpyHostToDevice, s);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

int hip_fail(hipError_t e) { return -static_cast<int>(e); }

}  // namespace

extern "C" miikv_status miikv_session_filename(uint64_t token_hash, uint32_t prefix_length, char* out,
                                               size_t out_cap) {
    if (out == nullptr) return MIIKV_EINVAL;
    const int n = std::snprintf(out, out_cap, "sess_%016llx_p%u.miinfer",
                                static_cast<unsigned long long>(token_hash), prefix_length);
    return (n < 0 || static_cast<size_t>(n) >= out_cap) ? MIIKV_EINVAL : MIIKV_OK;
}

extern "C" miikv_status miikv_session_save(const char* path, const char* model_id, const char* quantization,
                                           const uint32_t* tokens, uint32_t prefix_length,
                                           const miikv_view* kv_layers, uint32_t kv_layer_count, uint32_t seq,
                                           void* const* gdn_segments, const uint64_t* gdn_segment_bytes,
                                           uint32_t gdn_segment_count, void* stream) {
    const uint32_t P = prefix_length;
    Geometry g;
    if (path == nullptr || tokens == nullptr || P == 0 || gdn_segment_count % 2 != 0 ||
        (gdn_segment_count > 0 && (gdn_segments == nullptr || gdn_segment_bytes == nullptr)) ||
        !layers_geometry(kv_layers, kv_layer_count, P, g))
        return MIIKV_EINVAL;
    miikv_session_header h{};
    std::memcpy(h.magic, kMagic, 4);
    h.version = MIIKV_SESSION_VERSION;
    std::strncpy(h.model_id, model_id ? model_id : "", sizeof(h.model_id) - 1);
    std::strncpy(h.quantization, quantization ? quantization : "", sizeof(h.quantization) - 1);
    h.prefix_length = P;
    h.token_hash = miikv_token_hash(tokens, P);
    h.gdn_layers = gdn_segment_count / 2;
    h.gdn_state_bytes = sum_bytes(gdn_segment_bytes, gdn_segment_count);
    h.gqa_layers = kv_layer_count;
    h.kv_quant_mode = static_cast<uint8_t>(miikv_session_kv_mode(g.quant_mode));
    h.kv_bytes = g.layer_bytes * kv_layer_count;
    h.tokens_bytes = static_cast<uint64_t>(P) * sizeof(uint32_t);
    h.created_timestamp = static_cast<uint64_t>(std::time(nullptr));

    hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<uint8_t> gdn(h.gdn_state_bytes), kv(h.kv_bytes);
    uint64_t off = 0;
    for (uint32_t i = 0; i < gdn_segment_count; ++i) {
        if (gdn_segment_bytes[i] == 0) continue;
        hipError_t e = hipMemcpyAsync(gdn.data() + off, gdn_segments[i], gdn_segment_bytes[i],
                                      hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) return hip_fail(e);
        off += gdn_segment_bytes[i];
    }
    Staging st;
    if (hipError_t e = st.alloc(P, g); e != hipSuccess) return hip_fail(e);
    for (uint32_t l = 0; l < kv_layer_count; ++l) {
        const int r = miikv_export_canonical(&kv_layers[l], seq, 0, P, st.kc, st.ks, st.vc, st.vs, stream);
        if (r != MIIKV_OK) return r;
        if (hipError_t e = move_layer(st, g, P, kv.data() + g.layer_bytes * l, true, s); e != hipSuccess)
            return hip_fail(e);
        // the staging buffer is reused by the next layer
        if (hipError_t e = hipStreamSynchronize(s); e != hipSuccess) return hip_fail(e);
    }
    if (hipError_t e = hipStreamSynchronize(s); e != hipSuccess) return hip_fail(e);

    std::error_code ec;
    const std::filesystem::path final_path(path);
    if (final_path.has_parent_path()) std::filesystem::create_directories(final_path.parent_path(), ec);
    const std::string tmp = final_path.string() + ".tmp";
    {
        std::ofstream out(tmp, std::ios::binary | std::ios::trunc);
        if (!out.is_open()) return MIIKV_EINVAL;
        out.write(reinterpret_cast<const char*>(&h), sizeof(h));
        out.write(reinterpret_cast<const char*>(tokens), static_cast<std::streamsize>(h.tokens_bytes));
        out.write(reinterpret_cast<const char*>(gdn.data()), static_cast<std::streamsize>(gdn.size()));
        out.write(reinterpret_cast<const char*>(kv.data()), static_cast<std::streamsize>(kv.size()));
        out.flush();
        if (!out.good()) return MIIKV_EINVAL;
    }
    std::filesystem::rename(tmp, final_path, ec);
    return ec ? MIIKV_EINVAL : MIIKV_OK;
}

extern "C" int miikv_session_inspect(const char* path, miikv_session_header* out, uint32_t* tokens_out,
                                     uint32_t tokens_cap) {
    if (path == nullptr || out == nullptr) return 0;
    std::ifstream in(path, std::ios::binary);
    if (!in.is_open()) return 0;
    if (!in.read(reinterpret_cast<char*>(out), sizeof(*out))) return 0;
    if (std::memcmp(out->magic, kMagic, 4) != 0 || out->version != MIIKV_SESSION_VERSION) return 0;
    if (tokens_out != nullptr && out->prefix_length > 0) {
        if (out->prefix_length > tokens_cap ||
            out->tokens_bytes != static_cast<uint64_t>(out->prefix_length) * sizeof(uint32_t))
            return 0;
        if (!in.read(reinterpret_cast<char*>(tokens_out), static_cast<std::streamsize>(out->tokens_bytes))) return 0;
    }
    return 1;
}

extern "C" int miikv_session_load(const char* path, const char* model_id, const char* quantization,
                                  const miikv_view* kv_layers, uint32_t kv_layer_count, uint32_t seq,
                                  void* const* gdn_segments, const uint64_t* gdn_segment_bytes,
                                  uint32_t gdn_segment_count, uint32_t* tokens_out, uint32_t tokens_cap,
                                  uint32_t* prefix_length_out, void* stream) {
    if (path == nullptr || tokens_out == nullptr || prefix_length_out == nullptr) return 0;
    if (gdn_segment_count > 0 && (gdn_segments == nullptr || gdn_segment_bytes == nullptr)) return 0;
    std::ifstream in(path, std::ios::binary);
    if (!in.is_open()) return 0;
    miikv_session_header h{};
    if (!in.read(reinterpret_cast<char*>(&h), sizeof(h))) return 0;
    if (std::memcmp(h.magic, kMagic, 4) != 0 || h.version != MIIKV_SESSION_VERSION) return 0;
    if (field(h.model_id, sizeof(h.model_id)) != (model_id ? model_id : "") ||
        field(h.quantization, sizeof(h.quantization)) != (quantization ? quantization : ""))
        return 0;
    const uint32_t P = h.prefix_length;
    Geometry g;
    if (P == 0 || P > tokens_cap || h.gdn_layers * 2 != gdn_segment_count || h.gqa_layers != kv_layer_count ||
        h.tokens_bytes != static_cast<uint64_t>(P) * 4 ||
        h.gdn_state_bytes != sum_bytes(gdn_segment_bytes, gdn_segment_count) ||
        !layers_geometry(kv_layers, kv_layer_count, P, g) || h.kv_bytes != g.layer_bytes * kv_layer_count ||
        h.kv_quant_mode != miikv_session_kv_mode(g.quant_mode))
        return 0;
    std::vector<uint32_t> tokens(P);
    std::vector<uint8_t> gdn(h.gdn_state_bytes), kv(h.kv_bytes);
    if (!in.read(reinterpret_cast<char*>(tokens.data()), static_cast<std::streamsize>(h.tokens_bytes)) ||
        !in.read(reinterpret_cast<char*>(gdn.data()), static_cast<std::streamsize>(gdn.size())) ||
        !in.read(reinterpret_cast<char*>(kv.data()), static_cast<std::streamsize>(kv.size())))
        return 0;
    if (miikv_token_hash(tokens.data(), P) != h.token_hash) return 0;

    hipStream_t s = static_cast<hipStream_t>(stream);
    uint64_t off = 0;
    for (uint32_t i = 0; i < gdn_segment_count; ++i) {
        if (gdn_segment_bytes[i] == 0) continue;
        hipError_t e = hipMemcpyAsync(gdn_segments[i], gdn.data() + off, gdn_segment_bytes[i],
                                      hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return hip_fail(e);
        off += gdn_segment_bytes[i];
    }
    Staging st;
    if (hipError_t e = st.alloc(P, g); e != hipSuccess) return hip_fail(e);
    for (uint32_t l = 0; l < kv_layer_count; ++l) {
        if (hipError_t e = move_layer(st, g, P, kv.data() + g.layer_bytes * l, false, s); e != hipSuccess)
            return hip_fail(e);
        const int r = miikv_import_canonical(&kv_layers[l], seq, 0, P, st.kc, st.ks, st.vc, st.vs, stream);
        if (r != MIIKV_OK) return r < 0 ? r : 0;
        if (hipError_t e = hipStreamSynchronize(s); e != hipSuccess) return hip_fail(e);
    }
    std::memcpy(tokens_out, tokens.data(), h.tokens_bytes);
    *prefix_length_out = P;
    return 1;
}

extern "C" int miikv_session_find(const char* session_dir, const char* model_id, const char* quantization,
                                  const uint32_t* prompt, size_t prompt_len, char* path_out, size_t path_cap,
                                  uint32_t* prefix_length_out) {
    if (session_dir == nullptr || path_out == nullptr || prefix_length_out == nullptr ||
        (prompt_len > 0 && prompt == nullptr))
        return 0;
    std::error_code ec;
    if (!std::filesystem::is_directory(session_dir, ec)) return 0;
    uint32_t best = 0;
    std::string best_path;
    std::vector<uint32_t> toks;
    for (const auto& entry : std::filesystem::directory_iterator(session_dir, ec)) {
        if (!entry.is_regular_file(ec) || entry.path().extension() != ".miinfer") continue;
        miikv_session_header h{};
        if (!miikv_session_inspect(entry.path().c_str(), &h, nullptr, 0)) continue;
        if (field(h.model_id, sizeof(h.model_id)) != (model_id ? model_id : "") ||
            field(h.quantization, sizeof(h.quantization)) != (quantization ? quantization : ""))
            continue;
        if (h.prefix_length == 0 || h.prefix_length > prompt_len || h.prefix_length <= best) continue;
        // A file shorter or longer than its header says cannot load: skip it (the
        // reference only reads the header here).
        const uint64_t want = sizeof(h) + h.tokens_bytes + h.gdn_state_bytes + h.kv_bytes;
        if (entry.file_size(ec) != want || ec) continue;
        toks.resize(h.prefix_length);
        if (!miikv_session_inspect(entry.path().c_str(), &h, toks.data(), h.prefix_length)) continue;
        if (std::memcmp(toks.data(), prompt, sizeof(uint32_t) * h.prefix_length) != 0) continue;
        best = h.prefix_length;
        best_path = entry.path().string();
    }
    if (best == 0 || best_path.size() + 1 > path_cap) return 0;
    std::memcpy(path_out, best_path.c_str(), best_path.size() + 1);
    *prefix_length_out = best;
    return 1;
}
