// Kernel-argument blocks shared by the host runtime (runtime.cpp) and the device code. Plain
// C++ with fixed-width types only, so the host side compiles without the HIP device headers.
#pragma once

#include <stdint.h>

#define MOEARC_KV_F32 0u
#define MOEARC_KV_F16 1u

// Largest number of sequences one decode launch carries in its kernel arguments; the host splits
// larger batches into several launches.
#define MOEARC_MAX_SEQS_PER_LAUNCH 64


// Partial results of a split decode, written by the split kernel when a sequence's span is split
// across work items (one work item = one split of one sequence) and combined by the merge kernel.
// Head-major, so the records of one query head are contiguous:
//   rec_o[(h * n_items + item) * 64 + d]   un-normalised output (f32)
//   rec_ml[(h * n_items + item) * 2 + 0/1] running max (log2 domain) / denominator (f32)
#define MOEARC_MERGE_THREADS 256

// Floats of the code object's fixed record array (moearc_decode_scratch, 8 MiB), which the
// allocation-free decode entry point uses in place of the context's workspace: n_heads * work items
// * 66 floats must fit (64 heads: up to 496 work items; the planner's default is at most 128).
#define MOEARC_DECODE_SCRATCH_FLOATS (1u << 21)

// Kernel arguments of the split-K decode that are not preloaded scalars (the leading kernel
// arguments carry the KV and block-table bases, q, sequence 0's span, split and item count, and
// the geometry). Passed by value; the per-sequence arrays let one launch serve a ragged batch.
// Work item `it` (one (sequence, split) pair) covers the work-groups it * nkb + kbi for every
// KV-head block kbi, so consecutive work-groups -- which the dispatcher places on consecutive XCDs
// -- take consecutive KV-head blocks of the same split.
struct DecodeArgs {
    const float *q;               // [n_seqs][n_heads][64] f32
    const uint32_t *block_tables; // row b at block_tables + b * bt_stride
    const float *sinks;           // [n_heads] or null
    void *out;                    // [n_seqs][n_heads][64], f32 or f16
    float *rec_o;                 // partial records (see above)
    float *rec_ml;
    uint64_t bt_stride;
    uint32_t n_items;             // work items of the launch (records per head)
    uint32_t out_f16;
    float scale_log2e;            // scale * log2(e)
    uint32_t n_seqs;
    uint32_t item_begin[MOEARC_MAX_SEQS_PER_LAUNCH + 1]; // first work item of each sequence; entries
                                                         // n_seqs .. the end: the work-item count
    uint32_t kv_begin[MOEARC_MAX_SEQS_PER_LAUNCH];       // key span [kv_begin, n_kv)
    uint32_t n_kv[MOEARC_MAX_SEQS_PER_LAUNCH];
    uint32_t split_len[MOEARC_MAX_SEQS_PER_LAUNCH];      // keys per split (a multiple of the chunk)
};

// The merge kernel's per-sequence item ranges (sequence 0's end is a preloaded argument). One
// spare entry keeps the kernel's argument block a multiple of 8 bytes, the host struct's size.
struct MergeArgs {
    uint32_t item_begin[MOEARC_MAX_SEQS_PER_LAUNCH + 2];
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
    uint16_t *out_lo;             // with f16 output: also f16(o - hi) here, the low half of the
                                  // chunk product's activation split (default kernels; else null)
    uint32_t pair_half;           // the grid is two work-groups per CU, i and i + pair_half sharing
                                  // one (the dispatcher's order): pair_half; otherwise 0
    float boost_a, boost_b;       // the second work-group of a pair keeps a raised issue priority
                                  // for boost_a * its chunks - boost_b * its partner's chunks
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

// ---- quantised matrix-vector products (matvec.hip) ----------------------------------------------
//
// The weight formats, by GGUF type id: bytes per block (BB), elements per block (BE) and elements
// per "piece" (PE) -- the share of a row one lane decodes at a time. A lane owns the pieces
// lane, lane + 64, ... of every row, so the activation values of its pieces stay in registers
// while it walks the rows; MOEARC_MV_PPL_MAX bounds its pieces per pass (a row with more is
// walked in several column slabs).
#define MOEARC_MV_MAX_SEG 32   // matrices (or projections) one launch carries
#define MOEARC_MV_MAX_WAVES 8

constexpr uint32_t moearc_mv_bb(uint32_t ty) {
    return ty == 0 ? 4u : ty == 1 ? 2u : ty == 8 ? 34u : ty == 12 ? 144u : ty == 13 ? 176u
         : ty == 14 ? 210u : ty == 39 ? 17u : 0u;
}
constexpr uint32_t moearc_mv_be(uint32_t ty) {
    return ty == 0 || ty == 1 ? 1u : ty == 8 || ty == 39 ? 32u : ty == 12 || ty == 13 || ty == 14 ? 256u : 0u;
}
constexpr uint32_t moearc_mv_pe(uint32_t ty) {
    return ty == 0 ? 8u : ty == 12 || ty == 13 || ty == 39 ? 32u : 16u;
}
// Largest pieces per lane per pass: activation registers (PPL * PE) stay at or under 128, so a
// wave keeps at least three waves per SIMD of occupancy.
constexpr uint32_t moearc_mv_ppl_max(uint32_t) {
    return 4u;
}
// 16-byte granules one lane stages per slab (a slab of 64 * PPL pieces, any byte alignment).
constexpr uint32_t moearc_mv_gmax(uint32_t ty, uint32_t ppl) {
    return (uint32_t) ((64ull * ppl * moearc_mv_pe(ty) * moearc_mv_bb(ty) / moearc_mv_be(ty) + 30u + 1023u) / 1024u);
}
// Bytes of one wave's staging buffer for slabs of `slab_bytes`: the granules a slab at any
// alignment spans, plus slack for reads that run past a piece.
constexpr uint32_t moearc_mv_wave_buf(uint64_t slab_bytes) {
    return (uint32_t) (((slab_bytes + 30u + 15u) / 16u) * 16u + 64u);
}

// Segment s covers work-groups [wg_end[s-1], wg_end[s]) and rows [0, rows[s]) of matrix w[s]:
// out[s][r] = sum_c W_s[r][c] * x[s][c] (+ bias[s][r] when bit s of bias_mask is set; bias[s]
// then points at the bias, else at any readable rows[s] floats).
struct MatvecArgs {
    const uint8_t *w[MOEARC_MV_MAX_SEG];
    const float *x[MOEARC_MV_MAX_SEG];
    const float *bias[MOEARC_MV_MAX_SEG];
    float *out[MOEARC_MV_MAX_SEG];
    uint32_t rows[MOEARC_MV_MAX_SEG];
    uint32_t wg_end[MOEARC_MV_MAX_SEG];
    uint64_t row_bytes;
    uint32_t n_seg;
    uint32_t n_cols;
    uint32_t n_pieces;     // pieces per row, ceil(n_cols / PE)
    uint32_t n_slabs;      // column slabs per row
    uint32_t rpw;          // consecutive rows per wave
    uint32_t x_in_lds;     // 1: the activation is staged once per work-group in LDS
    uint32_t x_lds_bytes;  // LDS bytes before the waves' staging buffers
    uint32_t wave_buf;     // LDS bytes of one wave's staging buffer
    uint32_t bias_mask;
    uint32_t res_mask;     // bit s: out[s][r] += the result (the residual add), else out[s][r] = it
};

// Chunk-form projections (matmul.hip, matmul2.hip): Y[t][r] = sum_c W[r][c] X[t][c] (+ bias[r]) for
// the n_tok tokens of a prompt chunk, W Q8_0 (8), F16 (1), Q4_K (12), Q5_K (13), Q6_K (14) or
// MXFP4 (39), X given as its f16 hi + lo split. One launch serves up to MOEARC_MM_MAX_SEG matrices
// of one weight type over the same X (a block's q, k and v): its row tiles (grid x) run over the
// segments in order.
#define MOEARC_MM_TOKENS 64    // tokens per work-group
#define MOEARC_MM_MAX_SEG 3
struct MatmulSeg {
    const uint8_t *w;
    const float *bias;         // [rows] or null
    float *y;                  // [n_tok][y_stride]
    uint64_t row_bytes;
    uint64_t part_off;         // split launches: this matrix's sums at part + z * part_stride + part_off
    uint32_t rows, y_stride;
    uint32_t tile_end;         // row tiles of the launch up to and including this matrix's
    uint32_t pad;
};
struct MatmulArgs {
    MatmulSeg seg[MOEARC_MM_MAX_SEG];
    const uint16_t *xh, *xl;   // [n_tok][cols] f16: x = hi + lo to within 2^-22 |x|
    const float *xs;           // [n_tok][cols / 32] block sums of x (Q4_K, Q5_K), else unread
    float *part;               // split launches (grid z > 1): slice z's sums, [t][r] per matrix
    uint64_t part_stride;      // floats per slice: the sum of n_tok * rows over the matrices
    uint32_t n_seg, cols, n_tok;
    uint32_t accumulate;       // 1: y[t][r] += the result (the residual add), else y[t][r] = it
    uint32_t kb_per;           // k-blocks (of 32) per k-slice: work-group z takes blocks kb_per * z ..
    uint32_t pad;
};
