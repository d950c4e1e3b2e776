// Host-side policy of the prefix-reuse path: the page pool with reference counts
// and copy-on-write fork planning for paged q8_0 caches, and the prefix
// fingerprint / match logic of ReusableContext.  Pure C++ (no device calls);
// the device work these plans describe runs through miikv_copy_pages,
// miikv_copy_segments and miikv_clone_state.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "miikv.h"

// ---------------------------------------------------------------------------
// Page pool: free list + per-page reference counts.  No reference counterpart:
// the reference keeps one contiguous cache per layer (kv_cache.cpp:10-39) and
// reuses a prefix by leaving it in place (src/prefill_v2/model.cpp:752-846).
// ---------------------------------------------------------------------------
struct miikv_pool {
    std::vector<uint32_t> refs;
    std::vector<int32_t> free_list;  // LIFO
};

extern "C" miikv_pool* miikv_pool_create(uint32_t num_pages) {
    if (num_pages == 0 || num_pages > 0x7fffffffu) return nullptr;
    miikv_pool* p = new (std::nothrow) miikv_pool;
    if (p == nullptr) return nullptr;
    p->refs.assign(num_pages, 0);
    p->free_list.reserve(num_pages);
    for (uint32_t i = num_pages; i > 0; --i) p->free_list.push_back(static_cast<int32_t>(i - 1));
    return p;
}

extern "C" void miikv_pool_destroy(miikv_pool* p) { delete p; }

extern "C" int32_t miikv_pool_alloc(miikv_pool* p) {
    if (p == nullptr || p->free_list.empty()) return -1;
    const int32_t page = p->free_list.back();
    p->free_list.pop_back();
    p->refs[static_cast<size_t>(page)] = 1;
    return page;
}

static bool valid_page(const miikv_pool* p, int32_t page) {
    return p != nullptr && page >= 0 && static_cast<size_t>(page) < p->refs.size();
}

extern "C" miikv_status miikv_pool_ref(miikv_pool* p, int32_t page) {
    if (!valid_page(p, page) || p->refs[static_cast<size_t>(page)] == 0) return MIIKV_EINVAL;
    ++p->refs[static_cast<size_t>(page)];
    return MIIKV_OK;
}

extern "C" miikv_status miikv_pool_unref(miikv_pool* p, int32_t page) {
    if (!valid_page(p, page) || p->refs[static_cast<size_t>(page)] == 0) return MIIKV_EINVAL;
    if (--p->refs[static_cast<size_t>(page)] == 0) p->free_list.push_back(page);
    return MIIKV_OK;
}

extern "C" uint32_t miikv_pool_refcount(const miikv_pool* p, int32_t page) {
    return valid_page(p, page) ? p->refs[static_cast<size_t>(page)] : 0u;
}

extern "C" uint32_t miikv_pool_free_pages(const miikv_pool* p) {
    return p == nullptr ? 0u : static_cast<uint32_t>(p->free_list.size());
}

static uint32_t pages_for(uint32_t tokens, uint32_t page_tokens) {
    return (tokens + page_tokens - 1) / page_tokens;
}

extern "C" miikv_status miikv_pool_fork(miikv_pool* p, const int32_t* parent_row, uint32_t row_capacity,
                                        uint32_t length, uint32_t page_tokens, int32_t* child_row,
                                        int32_t* copy_src, int32_t* copy_dst, uint32_t* n_copies) {
    if (p == nullptr || page_tokens == 0 || (length > 0 && (parent_row == nullptr || child_row == nullptr)) ||
        n_copies == nullptr)
        return MIIKV_EINVAL;
    *n_copies = 0;
    const uint32_t np = pages_for(length, page_tokens);
    if (np > row_capacity) return MIIKV_EINVAL;  // both rows hold row_capacity entries
    for (uint32_t i = 0; i < np; ++i)
        if (!valid_page(p, parent_row[i]) || p->refs[static_cast<size_t>(parent_row[i])] == 0) return MIIKV_EINVAL;
    const bool partial = (length % page_tokens) != 0;
    if (partial && (copy_src == nullptr || copy_dst == nullptr)) return MIIKV_EINVAL;
    int32_t fresh = -1;
    if (partial) {
        fresh = miikv_pool_alloc(p);
        if (fresh < 0) return MIIKV_EINVAL;  // pool exhausted: nothing was changed
    }
    for (uint32_t i = 0; i < np; ++i) {
        if (partial && i + 1 == np) {
            child_row[i] = fresh;
            copy_src[0] = parent_row[i];
            copy_dst[0] = fresh;
            *n_copies = 1;
        } else {
            child_row[i] = parent_row[i];
            ++p->refs[static_cast<size_t>(parent_row[i])];
        }
    }
    return MIIKV_OK;
}

// n forks of one parent in one call: child i's row goes to child_rows + i*row_stride;
// copy_src/copy_dst (capacity n) receive the copy-on-write page pairs, *n_copies
// their count.  On pool exhaustion the forks made so far stay (each is complete)
// and MIIKV_EINVAL is returned with *n_done set.
extern "C" miikv_status miikv_pool_fork_n(miikv_pool* p, const int32_t* parent_row, uint32_t length,
                                          uint32_t page_tokens, uint32_t n, int32_t* child_rows, uint32_t row_stride,
                                          int32_t* copy_src, int32_t* copy_dst, uint32_t* n_copies,
                                          uint32_t* n_done) {
    if (p == nullptr || n_copies == nullptr || n_done == nullptr || page_tokens == 0 ||
        (n > 0 && child_rows == nullptr) || row_stride < pages_for(length, page_tokens))
        return MIIKV_EINVAL;
    *n_copies = 0;
    *n_done = 0;
    if (n == 0) return MIIKV_OK;
    const uint32_t np = pages_for(length, page_tokens);
    if (np > 0 && parent_row == nullptr) return MIIKV_EINVAL;
    for (uint32_t i = 0; i < np; ++i)
        if (!valid_page(p, parent_row[i]) || p->refs[static_cast<size_t>(parent_row[i])] == 0) return MIIKV_EINVAL;
    const bool partial = (length % page_tokens) != 0;
    if (partial && (copy_src == nullptr || copy_dst == nullptr)) return MIIKV_EINVAL;
    // The forks that fit: each partial fork takes one fresh page.
    const uint32_t k = partial ? static_cast<uint32_t>(std::min<size_t>(n, p->free_list.size())) : n;
    // The full pages are shared by every child: one reference-count pass for all k.
    const uint32_t shared = partial ? np - 1 : np;
    for (uint32_t i = 0; i < shared; ++i) p->refs[static_cast<size_t>(parent_row[i])] += k;
    for (uint32_t c = 0; c < k; ++c) {
        int32_t* row = child_rows + static_cast<size_t>(c) * row_stride;
        if (shared > 0) std::memcpy(row, parent_row, shared * sizeof(int32_t));
        if (partial) {
            const int32_t fresh = miikv_pool_alloc(p);  // cannot fail: k <= free pages
            row[np - 1] = fresh;
            copy_src[c] = parent_row[np - 1];
            copy_dst[c] = fresh;
        }
    }
    *n_copies = partial ? k : 0;
    *n_done = k;
    return k == n ? MIIKV_OK : MIIKV_EINVAL;
}

extern "C" miikv_status miikv_pool_prepare_append(miikv_pool* p, int32_t* row, uint32_t row_capacity,
                                                  uint32_t position, uint32_t page_tokens, int32_t* copy_src,
                                                  int32_t* copy_dst, uint32_t* n_copies) {
    if (p == nullptr || row == nullptr || page_tokens == 0 || n_copies == nullptr) return MIIKV_EINVAL;
    *n_copies = 0;
    const uint32_t i = position / page_tokens;
    if (i >= row_capacity) return MIIKV_EINVAL;
    if (position % page_tokens == 0 && row[i] < 0) {
        // First token of a new page: allocate it (a shared full page is never written).
        // An entry that already names a page (a repeated call) is handled below, so the
        // page it holds is neither leaked nor replaced.
        const int32_t fresh = miikv_pool_alloc(p);
        if (fresh < 0) return MIIKV_EINVAL;
        row[i] = fresh;
        return MIIKV_OK;
    }
    if (!valid_page(p, row[i]) || p->refs[static_cast<size_t>(row[i])] == 0) return MIIKV_EINVAL;
    if (p->refs[static_cast<size_t>(row[i])] == 1) return MIIKV_OK;  // exclusively owned
    if (copy_src == nullptr || copy_dst == nullptr) return MIIKV_EINVAL;
    const int32_t fresh = miikv_pool_alloc(p);
    if (fresh < 0) return MIIKV_EINVAL;
    copy_src[0] = row[i];
    copy_dst[0] = fresh;
    *n_copies = 1;
    --p->refs[static_cast<size_t>(row[i])];
    row[i] = fresh;
    return MIIKV_OK;
}

// Drops the row's page references and marks its entries -1, so that a row reused
// after release cannot hand prepare_append a page id that may since belong to
// another sequence.
extern "C" miikv_status miikv_pool_release(miikv_pool* p, int32_t* row, uint32_t length, uint32_t page_tokens) {
    if (p == nullptr || page_tokens == 0 || (length > 0 && row == nullptr)) return MIIKV_EINVAL;
    const uint32_t np = pages_for(length, page_tokens);
    for (uint32_t i = 0; i < np; ++i)
        if (!valid_page(p, row[i]) || p->refs[static_cast<size_t>(row[i])] == 0) return MIIKV_EINVAL;
    for (uint32_t i = 0; i < np; ++i) {
        miikv_pool_unref(p, row[i]);
        row[i] = -1;
    }
    return MIIKV_OK;
}

// ---------------------------------------------------------------------------
// Prefix fingerprint and match policy: restates ReusableContext
// (include/miinfer/prefill_v2/reusable_context.hpp:17-129,
//  src/prefill_v2/reusable_context.cpp:130-207).
// ---------------------------------------------------------------------------
struct miikv_prefix_ctx {
    std::string model_id;
    std::string quantization;
    uint32_t prefix_length = 0;
    uint64_t token_hash = 0;
    uint32_t layout_version = MIIKV_STATE_LAYOUT_VERSION;
    std::vector<uint32_t> tokens;
    bool state_valid = false;  // a state checkpoint was captured with the prefix
};

// 64-bit FNV-1a over u32 tokens widened to u64 (reusable_context.hpp:38-45).
extern "C" uint64_t miikv_token_hash(const uint32_t* tokens, size_t count) {
    uint64_t hash = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < count; ++i) {
        hash ^= static_cast<uint64_t>(tokens[i]);
        hash *= 0x100000001b3ull;
    }
    return hash;
}

extern "C" miikv_prefix_ctx* miikv_prefix_create(const char* model_id, const char* quantization) {
    miikv_prefix_ctx* c = new (std::nothrow) miikv_prefix_ctx;
    if (c == nullptr) return nullptr;
    c->model_id = model_id ? model_id : "";
    c->quantization = quantization ? quantization : "";
    return c;
}

extern "C" void miikv_prefix_destroy(miikv_prefix_ctx* c) { delete c; }

extern "C" void miikv_prefix_clear(miikv_prefix_ctx* c) {
    if (c == nullptr) return;
    c->state_valid = false;
    c->tokens.clear();
    c->prefix_length = 0;
    c->token_hash = 0;
}

// save (reusable_context.cpp:138-153): an empty prefix clears; otherwise the caller
// has captured the recurrent state (capture = miikv_copy_segments) and the
// fingerprint is recorded.
extern "C" miikv_status miikv_prefix_save(miikv_prefix_ctx* c, const uint32_t* tokens, size_t count) {
    if (c == nullptr || (count > 0 && tokens == nullptr) || count > 0xffffffffu) return MIIKV_EINVAL;
    if (count == 0) {
        miikv_prefix_clear(c);
        return MIIKV_OK;
    }
    c->tokens.assign(tokens, tokens + count);
    c->prefix_length = static_cast<uint32_t>(count);
    c->token_hash = miikv_token_hash(tokens, count);
    c->layout_version = MIIKV_STATE_LAYOUT_VERSION;
    c->state_valid = true;
    return MIIKV_OK;
}

// check_match (reusable_context.cpp:155-185): precedence Empty -> Version -> Model ->
// Quantization -> PromptShorter -> token compare.
extern "C" int miikv_prefix_check(const miikv_prefix_ctx* c, const uint32_t* prompt, size_t count,
                                  const char* model_id, const char* quantization) {
    if (c == nullptr || !c->state_valid || c->prefix_length == 0) return MIIKV_MATCH_EMPTY_CACHE;
    if (c->layout_version != MIIKV_STATE_LAYOUT_VERSION) return MIIKV_MATCH_VERSION_MISMATCH;
    if (c->model_id != (model_id ? model_id : "")) return MIIKV_MATCH_MODEL_MISMATCH;
    if (c->quantization != (quantization ? quantization : "")) return MIIKV_MATCH_QUANTIZATION_MISMATCH;
    if (count < c->prefix_length) return MIIKV_MATCH_PROMPT_SHORTER;
    if (prompt == nullptr) return MIIKV_MATCH_PREFIX_MISMATCH;
    if (std::memcmp(prompt, c->tokens.data(), sizeof(uint32_t) * c->prefix_length) != 0)
        return MIIKV_MATCH_PREFIX_MISMATCH;
    return MIIKV_MATCH_EXACT;
}

extern "C" uint32_t miikv_prefix_length(const miikv_prefix_ctx* c) { return c ? c->prefix_length : 0u; }

extern "C" uint64_t miikv_prefix_hash(const miikv_prefix_ctx* c) { return c ? c->token_hash : 0u; }

extern "C" void miikv_prefix_set_layout_version(miikv_prefix_ctx* c, uint32_t version) {
    if (c) c->layout_version = version;
}

// ---------------------------------------------------------------------------
// Prefix registry: several saved prefixes over one page pool.  Each entry keeps
// the fingerprint of ReusableContext (model, quantization, layout version,
// tokens + FNV-1a hash; reusable_context.hpp:17-129) and holds one reference on
// every page of its page row, so its KV pages outlive the session that wrote
// them; forks share the full pages and copy the partial last page, as
// miikv_pool_fork does.  The reference keeps a single slot
// (reusable_context.cpp:130-207, used by model.cpp:752-871); the registry applies
// the same match rule to each entry and picks the longest matching prefix.
// ---------------------------------------------------------------------------
struct miikv_registry {
    struct Entry {
        uint32_t id;
        std::vector<uint32_t> tokens;
        uint64_t hash;
        uint32_t layout_version;
        std::vector<int32_t> pages;
        uint64_t tag;
        uint64_t last_use;
    };
    miikv_pool* pool = nullptr;
    uint32_t page_tokens = 0;
    uint32_t max_entries = 0;
    std::string model_id;
    std::string quantization;
    std::vector<Entry> entries;
    uint32_t next_id = 1;
    uint64_t clock = 0;

    Entry* find(uint32_t id) {
        for (auto& e : entries)
            if (e.id == id) return &e;
        return nullptr;
    }
    void drop(size_t i) {
        for (int32_t pg : entries[i].pages) miikv_pool_unref(pool, pg);
        entries.erase(entries.begin() + static_cast<std::ptrdiff_t>(i));
    }
};

extern "C" miikv_registry* miikv_registry_create(miikv_pool* pool, uint32_t page_tokens, uint32_t max_entries,
                                                 const char* model_id, const char* quantization) {
    if (pool == nullptr || page_tokens == 0 || max_entries == 0) return nullptr;
    miikv_registry* r = new (std::nothrow) miikv_registry;
    if (r == nullptr) return nullptr;
    r->pool = pool;
    r->page_tokens = page_tokens;
    r->max_entries = max_entries;
    r->model_id = model_id ? model_id : "";
    r->quantization = quantization ? quantization : "";
    return r;
}

extern "C" void miikv_registry_destroy(miikv_registry* r) {
    if (r == nullptr) return;
    while (!r->entries.empty()) r->drop(r->entries.size() - 1);
    delete r;
}

extern "C" uint32_t miikv_registry_count(const miikv_registry* r) {
    return r ? static_cast<uint32_t>(r->entries.size()) : 0u;
}

extern "C" miikv_status miikv_registry_save(miikv_registry* r, const uint32_t* tokens, uint32_t count,
                                            const int32_t* row, uint32_t row_capacity, uint64_t tag,
                                            uint32_t* entry_id_out) {
    if (r == nullptr || count == 0 || tokens == nullptr || row == nullptr || entry_id_out == nullptr)
        return MIIKV_EINVAL;
    const uint32_t np = pages_for(count, r->page_tokens);
    if (np > row_capacity) return MIIKV_EINVAL;
    for (uint32_t i = 0; i < np; ++i)
        if (!valid_page(r->pool, row[i]) || r->pool->refs[static_cast<size_t>(row[i])] == 0) return MIIKV_EINVAL;
    // The same token sequence again: refresh the existing entry (its pages hold the
    // same prefix), do not store a second copy.
    const uint64_t hash = miikv_token_hash(tokens, count);
    for (auto& e : r->entries) {
        if (e.tokens.size() == count && e.hash == hash &&
            std::memcmp(e.tokens.data(), tokens, sizeof(uint32_t) * count) == 0) {
            e.last_use = ++r->clock;
            *entry_id_out = e.id;
            return MIIKV_OK;
        }
    }
    if (r->entries.size() >= r->max_entries) return MIIKV_EWORKSPACE;  // full: evict first
    miikv_registry::Entry e;
    e.id = r->next_id++;
    e.tokens.assign(tokens, tokens + count);
    e.hash = hash;
    e.layout_version = MIIKV_STATE_LAYOUT_VERSION;
    e.pages.assign(row, row + np);
    e.tag = tag;
    e.last_use = ++r->clock;
    for (int32_t pg : e.pages) miikv_pool_ref(r->pool, pg);
    *entry_id_out = e.id;
    r->entries.push_back(std::move(e));
    return MIIKV_OK;
}

// The ReusableContext::check_match rule for one entry (reusable_context.cpp:155-185).
static int registry_check(const miikv_registry& r, const miikv_registry::Entry& e, const uint32_t* prompt,
                          uint32_t count, const char* model_id, const char* quantization) {
    if (e.layout_version != MIIKV_STATE_LAYOUT_VERSION) return MIIKV_MATCH_VERSION_MISMATCH;
    if (r.model_id != (model_id ? model_id : "")) return MIIKV_MATCH_MODEL_MISMATCH;
    if (r.quantization != (quantization ? quantization : "")) return MIIKV_MATCH_QUANTIZATION_MISMATCH;
    if (count < e.tokens.size()) return MIIKV_MATCH_PROMPT_SHORTER;
    if (prompt == nullptr || std::memcmp(prompt, e.tokens.data(), sizeof(uint32_t) * e.tokens.size()) != 0)
        return MIIKV_MATCH_PREFIX_MISMATCH;
    return MIIKV_MATCH_EXACT;
}

extern "C" int miikv_registry_lookup(const miikv_registry* r, const uint32_t* prompt, uint32_t count,
                                     const char* model_id, const char* quantization, uint32_t strict,
                                     uint32_t* entry_id_out, uint32_t* prefix_length_out) {
    if (entry_id_out) *entry_id_out = 0;
    if (prefix_length_out) *prefix_length_out = 0;
    if (r == nullptr || r->entries.empty()) return MIIKV_MATCH_EMPTY_CACHE;
    const miikv_registry::Entry* best = nullptr;
    const miikv_registry::Entry* recent = nullptr;
    int recent_result = MIIKV_MATCH_EMPTY_CACHE;
    for (const auto& e : r->entries) {
        int res = registry_check(*r, e, prompt, count, model_id, quantization);
        // strict: the prefix must leave at least one prompt token to run (model.cpp:758-763)
        if (res == MIIKV_MATCH_EXACT && strict && e.tokens.size() >= count) res = MIIKV_MATCH_PROMPT_SHORTER;
        if (res == MIIKV_MATCH_EXACT) {
            if (best == nullptr || e.tokens.size() > best->tokens.size()) best = &e;
        } else if (recent == nullptr || e.last_use > recent->last_use) {
            recent = &e;
            recent_result = res;
        }
    }
    if (best == nullptr) return recent_result;  // the most recently used entry's verdict
    if (entry_id_out) *entry_id_out = best->id;
    if (prefix_length_out) *prefix_length_out = static_cast<uint32_t>(best->tokens.size());
    return MIIKV_MATCH_EXACT;
}

extern "C" miikv_status miikv_registry_fork(miikv_registry* r, uint32_t entry_id, int32_t* child_row,
                                            uint32_t row_capacity, int32_t* copy_src, int32_t* copy_dst,
                                            uint32_t* n_copies) {
    if (r == nullptr) return MIIKV_EINVAL;
    miikv_registry::Entry* e = r->find(entry_id);
    if (e == nullptr) return MIIKV_EINVAL;
    if (row_capacity < e->pages.size()) return MIIKV_EINVAL;
    const miikv_status st = miikv_pool_fork(r->pool, e->pages.data(), static_cast<uint32_t>(e->pages.size()),
                                            static_cast<uint32_t>(e->tokens.size()), r->page_tokens, child_row,
                                            copy_src, copy_dst, n_copies);
    if (st == MIIKV_OK) e->last_use = ++r->clock;
    return st;
}

extern "C" miikv_status miikv_registry_release(miikv_registry* r, uint32_t entry_id, uint64_t* tag_out) {
    if (r == nullptr) return MIIKV_EINVAL;
    for (size_t i = 0; i < r->entries.size(); ++i) {
        if (r->entries[i].id == entry_id) {
            if (tag_out) *tag_out = r->entries[i].tag;
            r->drop(i);
            return MIIKV_OK;
        }
    }
    return MIIKV_EINVAL;
}

extern "C" miikv_status miikv_registry_evict_lru(miikv_registry* r, uint32_t* entry_id_out, uint64_t* tag_out) {
    if (r == nullptr || r->entries.empty()) return MIIKV_EINVAL;
    size_t lru = 0;
    for (size_t i = 1; i < r->entries.size(); ++i)
        if (r->entries[i].last_use < r->entries[lru].last_use) lru = i;
    if (entry_id_out) *entry_id_out = r->entries[lru].id;
    if (tag_out) *tag_out = r->entries[lru].tag;
    r->drop(lru);
    return MIIKV_OK;
}

extern "C" miikv_status miikv_registry_info(const miikv_registry* r, uint32_t entry_id, uint32_t* length,
                                            uint64_t* token_hash, uint64_t* tag, int32_t* pages,
                                            uint32_t pages_cap) {
    if (r == nullptr) return MIIKV_EINVAL;
    for (const auto& e : r->entries) {
        if (e.id != entry_id) continue;
        if (length) *length = static_cast<uint32_t>(e.tokens.size());
        if (token_hash) *token_hash = e.hash;
        if (tag) *tag = e.tag;
        if (pages) {
            if (pages_cap < e.pages.size()) return MIIKV_EINVAL;
            std::memcpy(pages, e.pages.data(), sizeof(int32_t) * e.pages.size());
        }
        return MIIKV_OK;
    }
    return MIIKV_EINVAL;
}

extern "C" miikv_status miikv_registry_set_layout_version(miikv_registry* r, uint32_t entry_id, uint32_t version) {
    if (r == nullptr) return MIIKV_EINVAL;
    miikv_registry::Entry* e = r->find(entry_id);
    if (e == nullptr) return MIIKV_EINVAL;
    e->layout_version = version;
    return MIIKV_OK;
}
