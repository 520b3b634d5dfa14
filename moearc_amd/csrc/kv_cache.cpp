// Host-side KV page pool and cache geometry (include/moearc_kv.h).
//
// The pool follows PagedKvCache (crates/moearc-engine/src/kv.rs:85-205): a free list popped from
// the back (page 0 first on a fresh pool; a freed page is reused before any other), one page
// table per sequence, pages taken only as tokens need them, and every refusal leaving the pool
// exactly as it was. Differences, both deliberate: begin() on a sequence that is already active
// is refused (-2) where the reference's HashMap insert would drop its pages on the floor; and the
// chunk append (a prefill chunk's places in one all-or-nothing call) is this build's addition.
#include "moearc_kv.h"

#include <algorithm>
#include <new>
#include <unordered_map>
#include <vector>

namespace {

constexpr int kOk = 0, kNull = -1, kRange = -2;

struct SeqPages {
    std::vector<uint32_t> pages;  // logical order: token t lives in pages[t / page_tokens]
    uint32_t tokens = 0;          // tokens written so far
};

uint32_t div_ceil(uint64_t a, uint64_t b) { return (uint32_t) ((a + b - 1) / b); }

}  // namespace

struct moearc_kv_pool {
    uint32_t page_tokens = 0, context_limit = 0, total_pages = 0;
    std::vector<uint32_t> free;
    std::unordered_map<uint64_t, SeqPages> seqs;
    int err = 0;
    uint32_t err_a = 0, err_b = 0;

    int fail(int code, uint32_t a = 0, uint32_t b = 0) {
        err = code;
        err_a = a;
        err_b = b;
        return code;
    }
    int ok() { return fail(kOk); }
};

extern "C" {

int moearc_kv_pool_create(uint32_t total_pages, uint32_t page_tokens, uint32_t context_limit,
                          moearc_kv_pool **out) {
    if (!out) return kNull;
    *out = nullptr;
    if (total_pages == 0 || page_tokens == 0) return MOEARC_KV_INVALID_GEOMETRY;
    moearc_kv_pool *p = new (std::nothrow) moearc_kv_pool;
    if (!p) return kNull;
    p->page_tokens = page_tokens;
    p->context_limit = context_limit;
    p->total_pages = total_pages;
    p->free.resize(total_pages);
    for (uint32_t i = 0; i < total_pages; ++i) p->free[i] = total_pages - 1u - i;  // pop() -> 0 first
    *out = p;
    return kOk;
}

void moearc_kv_pool_destroy(moearc_kv_pool *p) { delete p; }

int moearc_kv_pool_last_error(const moearc_kv_pool *p, uint32_t *a, uint32_t *b) {
    if (!p) return kNull;
    if (a) *a = p->err_a;
    if (b) *b = p->err_b;
    return p->err;
}

int moearc_kv_pool_begin(moearc_kv_pool *p, uint64_t seq, uint32_t prompt_tokens) {
    if (!p) return kNull;
    if (prompt_tokens > p->context_limit)
        return p->fail(MOEARC_KV_CONTEXT_LIMIT, prompt_tokens, p->context_limit);
    if (p->seqs.count(seq)) return p->fail(kRange);
    const uint32_t needed = div_ceil(prompt_tokens, p->page_tokens);
    if (needed > p->free.size()) return p->fail(MOEARC_KV_EXHAUSTED, needed, (uint32_t) p->free.size());
    SeqPages s;
    s.pages.reserve(needed);
    for (uint32_t i = 0; i < needed; ++i) {
        s.pages.push_back(p->free.back());
        p->free.pop_back();
    }
    s.tokens = prompt_tokens;
    p->seqs.emplace(seq, std::move(s));
    return p->ok();
}

// n more tokens for `seq`, all or nothing; places written to pages/slots when non-null.
static int append_n(moearc_kv_pool *p, uint64_t seq, uint32_t n, uint32_t *pages, uint32_t *slots) {
    auto it = p->seqs.find(seq);
    if (it == p->seqs.end()) return p->fail(MOEARC_KV_UNKNOWN_SEQUENCE);
    SeqPages &s = it->second;
    const uint64_t want = (uint64_t) s.tokens + n;
    if (want > p->context_limit)
        return p->fail(MOEARC_KV_CONTEXT_LIMIT, n == 1 ? s.tokens : (uint32_t) std::min<uint64_t>(want, 0xFFFFFFFFu),
                       p->context_limit);
    const uint32_t have = (uint32_t) s.pages.size();
    const uint32_t need_total = div_ceil(want, p->page_tokens);
    const uint32_t extra = need_total > have ? need_total - have : 0u;
    if (extra > p->free.size()) return p->fail(MOEARC_KV_EXHAUSTED, extra, (uint32_t) p->free.size());
    for (uint32_t i = 0; i < extra; ++i) {  // pages are taken before the sequence changes
        s.pages.push_back(p->free.back());
        p->free.pop_back();
    }
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t t = s.tokens + i;
        if (pages) pages[i] = s.pages[t / p->page_tokens];
        if (slots) slots[i] = t % p->page_tokens;
    }
    s.tokens += n;
    return p->ok();
}

int moearc_kv_pool_append(moearc_kv_pool *p, uint64_t seq, uint32_t *page, uint32_t *slot) {
    if (!p) return kNull;
    return append_n(p, seq, 1, page, slot);
}

int moearc_kv_pool_append_chunk(moearc_kv_pool *p, uint64_t seq, uint32_t n, uint32_t *pages,
                                uint32_t *slots) {
    if (!p || (n && (!pages || !slots))) return kNull;
    return append_n(p, seq, n, pages, slots);
}

int moearc_kv_pool_end(moearc_kv_pool *p, uint64_t seq, uint32_t *n_pages) {
    if (!p) return kNull;
    auto it = p->seqs.find(seq);
    if (it == p->seqs.end()) return p->fail(MOEARC_KV_UNKNOWN_SEQUENCE);
    const std::vector<uint32_t> &pg = it->second.pages;
    if (n_pages) *n_pages = (uint32_t) pg.size();
    for (auto r = pg.rbegin(); r != pg.rend(); ++r) p->free.push_back(*r);
    p->seqs.erase(it);
    return p->ok();
}

int moearc_kv_pool_pages(const moearc_kv_pool *p, uint64_t seq, uint32_t *pages, uint32_t cap,
                         uint32_t *n_pages, uint32_t *tokens) {
    if (!p) return kNull;
    auto it = p->seqs.find(seq);
    if (it == p->seqs.end()) return MOEARC_KV_UNKNOWN_SEQUENCE;
    const SeqPages &s = it->second;
    if (pages) std::copy_n(s.pages.begin(), std::min<size_t>(cap, s.pages.size()), pages);
    if (n_pages) *n_pages = (uint32_t) s.pages.size();
    if (tokens) *tokens = s.tokens;
    return kOk;
}

int moearc_kv_pool_can_admit(const moearc_kv_pool *p, uint32_t tokens) {
    if (!p) return 0;
    return tokens <= p->context_limit && div_ceil(tokens, p->page_tokens) <= p->free.size();
}

int moearc_kv_pool_usage(const moearc_kv_pool *p, moearc_kv_usage *out) {
    if (!p || !out) return kNull;
    uint32_t used = 0, slack = 0;
    for (const auto &kv : p->seqs) {
        const uint32_t n = (uint32_t) kv.second.pages.size();
        used += n;
        const uint64_t cap = (uint64_t) n * p->page_tokens;
        slack += cap > kv.second.tokens ? (uint32_t) (cap - kv.second.tokens) : 0u;
    }
    *out = moearc_kv_usage{p->total_pages, used, (uint32_t) p->seqs.size(), slack};
    return kOk;
}

int moearc_kv_pool_block_tables(const moearc_kv_pool *p, const uint64_t *seqs, uint32_t n_seqs,
                                uint32_t stride, uint32_t *table) {
    if (!p || (n_seqs && (!seqs || !table))) return kNull;
    for (uint32_t b = 0; b < n_seqs; ++b) {  // validate every row before writing any
        auto it = p->seqs.find(seqs[b]);
        if (it == p->seqs.end()) return MOEARC_KV_UNKNOWN_SEQUENCE;
        if (it->second.pages.size() > stride) return kRange;
    }
    for (uint32_t b = 0; b < n_seqs; ++b) {
        const std::vector<uint32_t> &pg = p->seqs.find(seqs[b])->second.pages;
        uint32_t *row = table + (uint64_t) b * stride;
        std::copy(pg.begin(), pg.end(), row);
        std::fill(row + pg.size(), row + stride, 0u);
    }
    return kOk;
}

int moearc_kv_geometry(uint32_t n_ctx, uint32_t page_tokens, uint32_t n_swa, uint32_t chunk,
                       uint32_t *pages, uint32_t *swa_pages) {
    if (!pages || !swa_pages) return kNull;
    if (page_tokens == 0) return MOEARC_KV_INVALID_GEOMETRY;
    const uint32_t full = std::max(1u, div_ceil(n_ctx, page_tokens));
    uint32_t ring = full;
    if (n_swa) {
        const uint64_t live = (uint64_t) n_swa + std::max(chunk, 1u) - 1u;  // window + rest of the chunk
        ring = std::min(full, std::max(1u, div_ceil(live, page_tokens)));
    }
    *pages = full;
    *swa_pages = ring;
    return kOk;
}

int moearc_kv_ring_table(uint32_t pages, uint32_t swa_pages, uint32_t *table) {
    if (pages && !table) return kNull;
    if (swa_pages == 0) return kRange;
    for (uint32_t i = 0; i < pages; ++i) table[i] = i % swa_pages;
    return kOk;
}

}  // extern "C"
