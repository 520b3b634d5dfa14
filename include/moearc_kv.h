/*
 * moearc_kv.h -- host-side KV page pool and cache geometry of libmoearc_attn.so: which pages a
 * sequence's tokens occupy, and how large the ring of a sliding-window layer must be. No device
 * memory is touched: a page is an index into the K/V pools the caller allocated, and the block
 * tables built here are what moearc_attn_decode / moearc_attn_prefill / moearc_kv_append_chunk
 * index.
 *
 * Counterparts in the reference (paths relative to the reference repo):
 *   the pool          -- PagedKvCache, crates/moearc-engine/src/kv.rs:85-205
 *   the geometry      -- KvGeometry::plan / ring_tokens, crates/moearc-engine/src/moe.rs:716-771
 *   the cyclic table  -- swa_block_table, crates/moearc-engine/src/moe.rs:1428-1438, :1506-1513
 * The chunk entry point (moearc_kv_pool_append_chunk) and the batched block table have no
 * counterpart there: the reference engine appends one token per step.
 *
 * Return codes: 0 success; -1 a null argument; -2 an argument out of range; and the pool's own
 * refusals, mirroring kv.rs's KvError (details through moearc_kv_pool_last_error):
 */
#ifndef MOEARC_KV_H
#define MOEARC_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOEARC_KV_EXHAUSTED (-3)        /* KvError::Exhausted: detail a = pages requested, b = free */
#define MOEARC_KV_UNKNOWN_SEQUENCE (-4) /* KvError::UnknownSequence */
#define MOEARC_KV_CONTEXT_LIMIT (-5)    /* KvError::ContextLimit: a = tokens, b = limit */
#define MOEARC_KV_INVALID_GEOMETRY (-6) /* KvError::InvalidGeometry: a pool with no pages, or
                                           a page holding no tokens */

typedef struct moearc_kv_pool moearc_kv_pool;

/* KvUsage (kv.rs:64-72). */
typedef struct {
    uint32_t total_pages;
    uint32_t used_pages;
    uint32_t sequences;
    uint32_t slack_tokens; /* allocated but unwritten token slots (the tail of each last page) */
} moearc_kv_usage;

/* PagedKvCache::new (kv.rs:96-113): total_pages pages of page_tokens tokens each; a sequence may
 * hold at most context_limit tokens. Page 0 is handed out first on a fresh pool, and a freed
 * page is reused before any other. *out = NULL on failure. */
int moearc_kv_pool_create(uint32_t total_pages, uint32_t page_tokens, uint32_t context_limit,
                          moearc_kv_pool **out);
void moearc_kv_pool_destroy(moearc_kv_pool *p);

/* The last refusal's code and details (0 when the last call succeeded). */
int moearc_kv_pool_last_error(const moearc_kv_pool *p, uint32_t *a, uint32_t *b);

/* PagedKvCache::begin (kv.rs:120-138): a sequence with room for prompt_tokens tokens (the
 * prompt counts as written). Refusals leave the pool unchanged. */
int moearc_kv_pool_begin(moearc_kv_pool *p, uint64_t seq, uint32_t prompt_tokens);

/* PagedKvCache::append (kv.rs:140-169): one more token; a page is taken only when the current
 * one is full. *page, *slot: where the token lives. An exhausted pool leaves the sequence as
 * it was. */
int moearc_kv_pool_append(moearc_kv_pool *p, uint64_t seq, uint32_t *page, uint32_t *slot);

/* n more tokens at once (a prefill chunk), all or nothing: pages[i], slots[i] receive token i's
 * place -- the page_ids / slots arrays moearc_kv_append_chunk takes. */
int moearc_kv_pool_append_chunk(moearc_kv_pool *p, uint64_t seq, uint32_t n, uint32_t *pages,
                                uint32_t *slots);

/* PagedKvCache::end (kv.rs:171-180): returns the sequence's pages to the pool (most recent
 * first in line for reuse). *n_pages = how many. */
int moearc_kv_pool_end(moearc_kv_pool *p, uint64_t seq, uint32_t *n_pages);

/* PagedKvCache::pages_of (kv.rs:182-185): the sequence's page table (up to cap entries copied to
 * pages), its length and its token count. */
int moearc_kv_pool_pages(const moearc_kv_pool *p, uint64_t seq, uint32_t *pages, uint32_t cap,
                         uint32_t *n_pages, uint32_t *tokens);

/* PagedKvCache::can_admit (kv.rs:187-192): 1 if begin(tokens) would succeed now, else 0. */
int moearc_kv_pool_can_admit(const moearc_kv_pool *p, uint32_t tokens);

/* PagedKvCache::usage (kv.rs:194-205). */
int moearc_kv_pool_usage(const moearc_kv_pool *p, moearc_kv_usage *out);

/* Block tables of n_seqs sequences, one row of `stride` entries each (row b at table + b*stride,
 * entries past a sequence's pages are 0): the block_tables argument of
 * moearc_attn_decode_batched. -2 if a sequence holds more than stride pages. */
int moearc_kv_pool_block_tables(const moearc_kv_pool *p, const uint64_t *seqs, uint32_t n_seqs,
                                uint32_t stride, uint32_t *table);

/* KvGeometry::plan (moe.rs:735-757) for a context of n_ctx tokens in pages of page_tokens:
 * *pages = pages a full-attention layer needs, *swa_pages = pages of a windowed layer's ring
 * (n_swa = 0: no window, *swa_pages = *pages). A chunk of `chunk` tokens is appended before it
 * is attended, so while its first query attends, the keys from that query's window start to the
 * chunk's last token are all live: the ring holds n_swa + chunk - 1 tokens (chunk = 1 for token
 * by token decode, the reference's case), rounded up to whole pages and capped at *pages. */
int moearc_kv_geometry(uint32_t n_ctx, uint32_t page_tokens, uint32_t n_swa, uint32_t chunk,
                       uint32_t *pages, uint32_t *swa_pages);

/* The cyclic table a windowed layer indexes instead of the sequence's block table
 * (moe.rs:1506-1513): table[i] = i % swa_pages for i < pages, so logical key j lands in ring
 * slot j % (swa_pages * page_tokens) and the kernels need no notion of a ring. */
int moearc_kv_ring_table(uint32_t pages, uint32_t swa_pages, uint32_t *table);

#ifdef __cplusplus
}
#endif

#endif /* MOEARC_KV_H */
