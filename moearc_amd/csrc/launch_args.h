// Kernel-argument blocks shared by the host runtime (runtime.cpp) and the device code. Plain
// C++ with fixed-width types only, so the host side compiles without the HIP device headers.
#pragma once

#include <stdint.h>

#define MOEARC_KV_F32 0u
#define MOEARC_KV_F16 1u

// Largest number of sequences one decode launch carries in its kernel arguments; the host splits
// larger batches into several launches.
#define MOEARC_MAX_SEQS_PER_LAUNCH 64


// Partial-result record of one decode work item (one split of one KV head of one sequence),
// written to the workspace when a KV head's span is split across work-groups:
//   [0, 16)          running max per query head of the group (log2 domain)
//   [16, 32)         running denominator per head
//   [32, 32 + 64*16) un-normalised output, [head][dim]
#define MOEARC_PARTIAL_FLOATS (32 + 64 * 16)

// Work-groups of the split merge per (sequence, query head): each combines 64 / MOEARC_MERGE_PARTS
// output channels.
#define MOEARC_MERGE_PARTS 4
#define MOEARC_MERGE_THREADS 256

// Kernel arguments of the split-K decode. Passed by value; the per-sequence arrays let one launch
// serve a ragged batch. Work item `it` (one (sequence, split) pair) covers the work-groups
// it * nkb + kbi for every KV-head block kbi, so consecutive work-groups -- which the dispatcher
// places on consecutive XCDs -- take consecutive KV-head blocks of the same split.
struct DecodeArgs {
    const float *q;               // [n_seqs][n_heads][64] f32
    const uint16_t *k_pages;      // f16 bits, [page][slot][kv_head][64]
    const uint16_t *v_pages;
    const uint32_t *block_tables; // row b at block_tables + b * bt_stride
    const float *sinks;           // [n_heads] or null
    void *out;                    // [n_seqs][n_heads][64], f32 or f16
    float *ws;                    // partial records, one per work-group
    uint32_t *counters;           // [sequence][KV-head block] arrival counts, zero between launches;
                                  // non-null: the last work-group of a block merges its splits
    uint64_t bt_stride;
    uint32_t n_heads;
    uint32_t n_kv_heads;
    uint32_t group;               // n_heads / n_kv_heads, at most 16
    uint32_t pt_shift;            // log2(page_tokens)
    uint32_t out_f16;
    float scale_log2e;            // scale * log2(e)
    uint32_t n_seqs;
    uint32_t nkb;                 // KV-head blocks per work item (KV heads / heads per work-group)
    uint32_t item_begin[MOEARC_MAX_SEQS_PER_LAUNCH + 1]; // first work item of each sequence; entries
                                                         // n_seqs .. the end: the work-item count
    uint32_t kv_begin[MOEARC_MAX_SEQS_PER_LAUNCH];       // key span [kv_begin, n_kv)
    uint32_t n_kv[MOEARC_MAX_SEQS_PER_LAUNCH];
    uint32_t split_len[MOEARC_MAX_SEQS_PER_LAUNCH];      // keys per split (a multiple of 32)
};

// General decode (any head_dim <= 1024, f32 or f16 KV, any page size, any group).
struct DecodeGeneralArgs {
    const float *q;
    const void *k_pages;
    const void *v_pages;
    const uint32_t *block_tables;
    const float *sinks;
    void *out;
    uint64_t bt_stride;
    uint32_t n_heads;
    uint32_t n_kv_heads;
    uint32_t head_dim;
    uint32_t page_tokens;
    uint32_t kv_type;
    uint32_t out_f16;
    float scale;
    uint32_t n_seqs;
    uint32_t kv_begin[MOEARC_MAX_SEQS_PER_LAUNCH];
    uint32_t n_kv[MOEARC_MAX_SEQS_PER_LAUNCH];
};

// Chunked prefill: query rows ((token, head) pairs of one KV head's group) per work-group and the
// work-group size.
#define MOEARC_PREFILL_ROWS 128        // precise (hi/lo weights) kernels
#define MOEARC_PREFILL_FAST_ROWS 256   // default kernels: 64 rows per wave
#define MOEARC_PREFILL_THREADS 256

// Chunked prefill over f16 paged KV, head_dim 64.
struct PrefillArgs {
    const uint16_t *q;            // [n_q][n_heads][64] f16
    const uint16_t *k_pages;
    const uint16_t *v_pages;
    const uint32_t *block_table;
    const float *sinks;
    void *out;                    // [n_q][n_heads][64] f32 or f16
    uint32_t n_q;
    uint32_t pos0;
    uint32_t n_swa;               // 0 = full causal
    uint32_t n_heads;
    uint32_t n_kv_heads;
    uint32_t group;               // 1, 2, 4 or 8
    uint32_t pt_shift;
    uint32_t out_f16;
    float scale_log2e;
    uint32_t n_qtiles;            // query tiles per KV head
};

// RoPE parameters (moearc_rope, moearc_rope_kv_append_chunk): theta_scale = freq_base^(-2/n_dims),
// computed on the host; neox selects the (p, p + n_dims/2) pairing, else (2p, 2p + 1).
// Heads per thread of the RoPE kernels (grid y runs over groups of this many heads).
constexpr uint32_t ROPE_HEADS = 4;

struct RopeParams {
    uint32_t n_dims;
    uint32_t neox;
    float theta_scale;
    float freq_scale;
    float ext_factor;
    float attn_factor;
    float corr_lo;
    float corr_hi;
};
