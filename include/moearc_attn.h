/*
 * moearc_attn.h -- C ABI of libmoearc_attn.so, the MI355X (gfx950) build of MoEArc's attention
 * hot path.
 *
 * Names, argument order, argument types and return codes are those of the reference's FFI
 * (crates/moearc-kernels/src/ffi.rs), so the reference's Rust wrapper binds this library by
 * linking it in place of libmoearc_kernels.so. Paths cited are relative to the reference repo.
 *
 * Return codes (ffi.rs:8-10, kernels.cpp:470-476):
 *    0  accepted. Kernels are enqueued on the context's stream and not waited for: "0" means
 *       the work was accepted, not that it completed. A device fault surfaces at the next
 *       moearc_sync or moearc_copy_d2h.
 *   -1  a null argument, or a HIP call failed.
 *   -2  an argument out of range; nothing was enqueued.
 *
 * Types: `unsigned long` is 64-bit (LP64), as in the reference (ffi.rs:263). kv_type is the GGUF
 * type id: 0 = f32, 1 = f16.
 *
 * Threading: one context = one HIP stream, in order; every entry point taking a context enqueues
 * on that stream. A context is not safe to share across threads (lib.rs:1251-1253).
 */
#ifndef MOEARC_ATTN_H
#define MOEARC_ATTN_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct moearc_ctx moearc_ctx;

/* ---- lifecycle and memory (ffi.rs:20-51; kernels.cpp:804-966) ------------------------------- */

/* ffi.rs:20, kernels.cpp:804-828. Opens a stream on the current HIP device and loads the
 * kernels' code object with hipModuleLoad. NULL when no device or the code object is missing.
 * MOEARC_PROFILE_EVENTS=1 brackets every tracked call with a HIP event pair (see the report);
 * MOEARC_PROFILE_KERNELS=1 also brackets every kernel launch inside a call, and untracked calls. */
moearc_ctx *moearc_ctx_create(void);
/* ffi.rs:21, kernels.cpp:830. Waits for the stream, then frees everything the context owns. */
void moearc_ctx_destroy(moearc_ctx *c);
/* ffi.rs:22, kernels.cpp:839. 1 if the context records per-launch device times. */
int moearc_profile_events_enabled(moearc_ctx *c);
/* ffi.rs:23, kernels.cpp:841-846. Forget recorded times. */
int moearc_profile_events_reset(moearc_ctx *c);
/* ffi.rs:24-28, kernels.cpp:852-871. One "key nanoseconds calls" line per key; waits for the
 * recorded launches. Every tracked call is recorded once, under one key, as the reference records
 * each submission: "attn_decode r{n_heads} m{head_dim}" for a whole decode call (split and merge
 * launches, windowed and full layers alike; kernels.cpp:1905-1916), "mvq {type} r{rows} m1",
 * "mvq_batched {type} r{rows} m{n_mat}" and "mv_generic r{rows} m1" (F32/F16 weights) for the
 * matvecs (kernels.cpp:1057-1111, :1168-1196); this library's own entry points under their names
 * ("attn_prefill r{n_heads} m{head_dim}", "attn_qkv {type} ...", ...). Entry points the reference
 * does not track (zero, add, kv_append, quantize_f16, rope, matvec_f32) add no key. With
 * MOEARC_PROFILE_KERNELS=1, kernels are also recorded on their own as "kernel {name} r.. m.." --
 * nested inside their call's bracket, so those keys must not be added to the call keys. */
int moearc_profile_events_report(moearc_ctx *c, char *out, unsigned long cap);
/* ffi.rs:29, kernels.cpp:879-882. Block until the stream drains; reports a device fault. */
int moearc_sync(moearc_ctx *c);
/* ffi.rs:30. dst[0..n) = 0.0f. */
int moearc_zero(moearc_ctx *c, float *dst, unsigned long n);
/* ffi.rs:31, kernels.cpp:884-892. */
int moearc_device_name(moearc_ctx *c, char *out, unsigned long cap);
/* ffi.rs:32, kernels.cpp:895-898. NULL on failure. 256-byte aligned. */
void *moearc_alloc_device(moearc_ctx *c, unsigned long bytes);
/* ffi.rs:33, kernels.cpp:900-902. Waits for the stream before freeing. */
void moearc_free_device(moearc_ctx *c, void *p);
/* ffi.rs:34-39, kernels.cpp:904-907. Blocking. */
int moearc_copy_h2d(moearc_ctx *c, void *dst, const void *src, unsigned long bytes);
/* ffi.rs:40-45, kernels.cpp:962-965. Enqueued; src must stay valid until the stream passes it. */
int moearc_copy_h2d_async(moearc_ctx *c, void *dst, const void *src, unsigned long bytes);
/* ffi.rs:46-51, kernels.cpp:909-912. Blocking; waits for everything enqueued before it. */
int moearc_copy_d2h(moearc_ctx *c, void *dst, const void *src, unsigned long bytes);

/* ---- f16 codec (ffi.rs:189-194, kernels.cpp:1727-1735) ----------------------------------------
 * dst[i] = binary16(src[i]), IEEE round-to-nearest-even, subnormals rounded, overflow to +-inf,
 * NaN kept NaN with payload 0x200 | mant>>13 (kernels.cpp:152-186). Bit-exact to the reference. */
int moearc_quantize_f16(moearc_ctx *c, void *dst, const float *src, unsigned long n);

/* ---- paged KV cache write (ffi.rs:204-216, kernels.cpp:1782-1799) -----------------------------
 * Writes one token's K and V (f32 [n_kv_heads][head_dim]) into page `page_id`, slot `slot` of the
 * pools, layout [page][slot][kv_head][head_dim], stored as kv_type (f16 by the codec above).
 * Refusals: null pointer -> -1; kv_type not 0/1, page_tokens == 0, slot >= page_tokens,
 * n_kv_heads == 0 or head_dim == 0 -> -2. */
int moearc_kv_append(moearc_ctx *c, void *k_pages, void *v_pages, const float *k, const float *v,
                     unsigned int page_id, unsigned int slot, unsigned long n_kv_heads,
                     unsigned long head_dim, unsigned long page_tokens, unsigned int kv_type);

/* ---- single-query paged attention (ffi.rs:218-234, kernels.cpp:1837-1919) ---------------------
 * For each query head h (KV head h / (n_heads / n_kv_heads)), over logical keys
 * j in [kv_begin, n_kv) read through block_table (page block_table[j / page_tokens], slot
 * j % page_tokens):
 *     s_j = scale * (q_h . K_j)
 *     out_h = sum_j e^(s_j - M) V_j / (e^(sink_h - M) + sum_j e^(s_j - M)),  M = max(sink_h, max s_j)
 * with the sink term dropped when `sinks` is NULL. q and out are f32 [n_heads][head_dim].
 * Refusals, in this order (kernels.cpp:1842-1852): any of c, out, q, k_pages, v_pages, block_table
 * null -> -1; kv_type not 0/1 -> -2; n_heads, n_kv_heads, head_dim, n_kv or page_tokens zero -> -2;
 * n_heads % n_kv_heads != 0 -> -2; kv_begin >= n_kv -> -2; head_dim > 1024 -> -2.
 * Paths: f16 KV with head_dim 64, a group of at most 16 heads and a power-of-two page size run the
 * split-K MFMA kernel; every other accepted shape runs a general f32 kernel. */
int moearc_attn_decode(moearc_ctx *c, float *out, const float *q, const void *k_pages,
                       const void *v_pages, const unsigned int *block_table, const float *sinks,
                       unsigned long n_heads, unsigned long n_kv_heads, unsigned long head_dim,
                       unsigned long kv_begin, unsigned long n_kv, unsigned long page_tokens,
                       float scale, unsigned int kv_type);

/* ---- extensions (no single counterpart in the reference; same conventions) -------------------- */

/* Output element type of the extensions below. */
#define MOEARC_OUT_F32 0u
#define MOEARC_OUT_F16 1u

/* Batched ragged decode: n_seqs independent moearc_attn_decode calls in one launch.
 * Sequence b reads q[b][n_heads][head_dim], writes out[b][n_heads][head_dim] (f32 or f16 by
 * out_type), attends [kv_begin[b], n_kv[b]) through block-table row
 * block_tables[b * bt_stride ...]. kv_begin and n_kv are HOST arrays of n_seqs entries (the
 * engine keeps sequence lengths on the host, moe.rs:1890-1912); every other pointer is device
 * memory. Each sequence must equal the single call with the same arguments.
 * Refusals: as moearc_attn_decode per sequence (an empty span in any sequence -> -2), plus
 * n_seqs == 0, out_type not 0/1, or bt_stride < ceil(n_kv[b] / page_tokens) -> -2. */
int moearc_attn_decode_batched(moearc_ctx *c, void *out, unsigned int out_type, const float *q,
                               const void *k_pages, const void *v_pages,
                               const unsigned int *block_tables, unsigned long bt_stride,
                               const unsigned int *kv_begin, const unsigned int *n_kv,
                               const float *sinks, unsigned long n_seqs, unsigned long n_heads,
                               unsigned long n_kv_heads, unsigned long head_dim,
                               unsigned long page_tokens, float scale, unsigned int kv_type);

/* Allocation-free decode. No counterpart in the reference: for callers that cannot allocate --
 * code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. The
 * arguments, refusals and results of moearc_attn_decode_batched (the same kernels, bit-identical
 * outputs), but the partial records of split spans go to a fixed 8 MiB array inside the code
 * object (MOEARC_DECODE_SCRATCH_FLOATS floats, one array per context on its device, held until the
 * context is destroyed) instead of the context's workspace, and no profiling event is recorded, so
 * the call makes no hipMalloc, hipFree, event or host allocation. Limit: n_heads x work items x 66
 * floats must fit the array (64 heads: up to 496 work items; the default split plan uses at most
 * 128); a larger call is refused with -2, checked for every launch of the call before anything is
 * enqueued. Calls of one context reuse the array in stream order; calls that overlap in time on one
 * context (e.g. graphs captured from it replayed on other streams concurrently) race. Nothing in the
 * array needs clearing between calls. */
int moearc_attn_decode_batched_noalloc(moearc_ctx *c, void *out, unsigned int out_type, const float *q,
                                       const void *k_pages, const void *v_pages,
                                       const unsigned int *block_tables, unsigned long bt_stride,
                                       const unsigned int *kv_begin, const unsigned int *n_kv,
                                       const float *sinks, unsigned long n_seqs, unsigned long n_heads,
                                       unsigned long n_kv_heads, unsigned long head_dim,
                                       unsigned long page_tokens, float scale, unsigned int kv_type);

/* Chunked prefill over a paged f16 KV cache. The chunk's n_q tokens sit at absolute positions
 * pos0 .. pos0+n_q-1 and their K/V are already in the cache (logical keys 0 .. pos0+n_q-1 through
 * block_table). Row i is, exactly, moearc_attn_decode at n_kv = pos0+i+1 with
 * kv_begin = (n_swa > 0 ? max(0, pos0+i+1-n_swa) : 0) -- the reference engine's prefill, one
 * decode per prompt token (moe.rs:1856-1862, moe.rs:2020-2027).
 * q: f16 [n_q][n_heads][head_dim]; out: [n_q][n_heads][head_dim] f32 or f16 by out_type.
 * Requires kv_type 1 (f16), head_dim 64, a group n_heads/n_kv_heads of 1, 2, 4 or 8 and a
 * power-of-two page_tokens; other shapes -> -2. */
int moearc_attn_prefill(moearc_ctx *c, void *out, unsigned int out_type, const void *q,
                        const void *k_pages, const void *v_pages, const unsigned int *block_table,
                        const float *sinks, unsigned long n_q, unsigned long pos0,
                        unsigned long n_swa, unsigned long n_heads, unsigned long n_kv_heads,
                        unsigned long head_dim, unsigned long page_tokens, float scale,
                        unsigned int kv_type);

/* Chunk append: writes n_tok tokens' K and V (f32 [n_tok][n_kv_heads][head_dim]) at
 * (page_ids[t], slots[t]) (device u32 arrays). Equal to n_tok moearc_kv_append calls in order
 * (moe.rs:2029-2042 once per token); two tokens naming the same slot are a caller error.
 * Refusals as moearc_kv_append (slot range is not checked on the host: slots are device data). */
int moearc_kv_append_chunk(moearc_ctx *c, void *k_pages, void *v_pages, const float *k,
                           const float *v, const unsigned int *page_ids, const unsigned int *slots,
                           unsigned long n_tok, unsigned long n_kv_heads, unsigned long head_dim,
                           unsigned long page_tokens, unsigned int kv_type);

/* Rotary position embedding, ffi.rs:236-252 / kernels.cpp:1399-1468 (ggml's rope_yarn):
 * dst, src f32 [n_tokens][n_heads][head_dim] (dst may equal src), pos i32 [n_tokens] (device).
 * Pairs (p, p + n_dims/2) when neox != 0, else (2p, 2p + 1), rotated by
 * theta = pos * freq_base^(-2p/n_dims) with YaRN interpolation (freq_scale, ext_factor, corr_lo,
 * corr_hi) and magnitude scale attn_factor (times 1 + 0.1 ln(1/freq_scale) when ext_factor != 0);
 * channels >= n_dims pass through. freq_scale 1, ext_factor 0, attn_factor 1 is plain RoPE.
 * Returns -1 on a null pointer; -2 when n_dims is 0, odd or larger than head_dim, or when
 * n_heads exceeds 262140 (the launch grid's limit); 0 (nothing enqueued) for zero tokens or heads. */
int moearc_rope(moearc_ctx *c, float *dst, const float *src, const int *pos,
                unsigned long n_tokens, unsigned long n_heads, unsigned long head_dim,
                unsigned long n_dims, float freq_base, float freq_scale, float ext_factor,
                float attn_factor, float corr_lo, float corr_hi, int neox);

/* Extension (no counterpart in the reference, which rotates K with moearc_rope and then appends
 * it with moearc_kv_append once per token, moe.rs:1987-2042): K rotated exactly as moearc_rope
 * would, then K and V written as moearc_kv_append_chunk would, in one pass over a prefill chunk.
 * k, v f32 [n_tok][n_kv_heads][head_dim]; pos i32 [n_tok]; page_ids, slots u32 [n_tok] (all
 * device). Refusals: those of moearc_rope, then those of moearc_kv_append_chunk. */
int moearc_rope_kv_append_chunk(moearc_ctx *c, void *k_pages, void *v_pages, const float *k,
                                const float *v, const int *pos, const unsigned int *page_ids,
                                const unsigned int *slots, unsigned long n_tok,
                                unsigned long n_kv_heads, unsigned long head_dim,
                                unsigned long page_tokens, unsigned long n_dims, float freq_base,
                                float freq_scale, float ext_factor, float attn_factor,
                                float corr_lo, float corr_hi, int neox, unsigned int kv_type);

/* ---- attention projections: matrix-vector products and the bias add ---------------------------
 * Weight formats by GGUF type id: 0 F32, 1 F16, 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K, 39 MXFP4, laid
 * out as ggml writes them (row-major, each row n_cols / block_elems blocks). All pointers are
 * device pointers; W may sit at any byte alignment. Results match the reference's f64 twin
 * (reference.rs:305-336) within 2 (n_cols/32 + 5) * 2^-24 * sum|w x| per row. */

/* ffi.rs:68-75, kernels.cpp:1046-1111: out[r] = sum_c W[r][c] x[c] for r < n_rows.
 * Refusals: null pointer -> -1; unknown type_id, n_cols not a whole number of blocks,
 * n_rows >= 2^32 or n_cols >= 2^31 -> -2. n_rows == 0 -> 0, nothing enqueued. */
int moearc_matvec_q(moearc_ctx *c, unsigned int type_id, float *out, const void *w,
                    const float *x, unsigned long n_rows, unsigned long n_cols);

/* ffi.rs:77-87, kernels.cpp:1146-1206: n_mat matrices of one type and shape in one launch;
 * matrix m reads x + m * x_stride (x_stride 0: one shared x) and writes out[m * n_rows ..]. w is a
 * HOST array of n_mat device pointers. Bit-identical to n_mat moearc_matvec_q calls.
 * Refusals: null c/out/w/x or a null w[m] -> -1; n_mat > 32, and those of moearc_matvec_q -> -2.
 * n_mat == 0 or n_rows == 0 -> 0. */
int moearc_matvec_q_batched(moearc_ctx *c, unsigned int type_id, float *out,
                            const void *const *w, unsigned int n_mat, const float *x,
                            unsigned long x_stride, unsigned long n_rows, unsigned long n_cols);

/* ffi.rs:97-103, kernels.cpp:1116-1135: moearc_matvec_q over f32 weights (w f32 [n_rows][n_cols]).
 * Refusals: null pointer -> -1. */
int moearc_matvec_f32(moearc_ctx *c, float *out, const float *w, const float *x,
                      unsigned long n_rows, unsigned long n_cols);

/* ffi.rs:167-173, kernels.cpp:1676-1683: out[i] = a[i] + b[i]; out may alias a or b.
 * Refusals: null pointer -> -1. n == 0 -> 0. */
int moearc_add(moearc_ctx *c, float *out, const float *a, const float *b, unsigned long n);

/* Calibration read. No counterpart in the reference: for measurements that set the attention
 * kernels' HBM traffic beside what a plain streaming read reaches on the device. Reads `bytes`
 * bytes at src (16-byte aligned, a multiple of 16 bytes) with every load of a lane in flight at
 * once, 64 KiB per work-group, and writes out[g] = the xor of the 32-bit words of the g-th 64 KiB
 * (ceil(bytes / 65536) words). Null pointer -> -1; bytes 0, not a multiple of 16 or a misaligned
 * src -> -2. */
int moearc_read_floor(moearc_ctx *c, unsigned int *out, const void *src, unsigned long bytes);

/* Calibration of the matrix cores. No counterpart in the reference: for measurements that set the
 * prefill kernels' MFMA utilisation beside the rate the device sustains on such data. n_wgs
 * work-groups of 4 waves; wave w takes eight 1 KiB operand blocks of f16 values at
 * src + 8 KiB * w (four A and four B operands of v_mfma_f32_32x32x16_f16, lane l holding bytes
 * 16 l .. 16 l + 15 of each) and runs four accumulator chains for `iters` rounds of two MFMAs each
 * (round i, chain c: A[(c + i) % 4] times B[(c + i) % 4]); out[w] = the sum of its accumulators
 * over all lanes. src holds n_wgs * 32 KiB. Null pointer -> -1; n_wgs 0 or above 2^29 - 1,
 * iters 0, not a multiple of 4 or above 2^30, or a misaligned src -> -2. */
int moearc_mfma_floor(moearc_ctx *c, float *out, const void *src, unsigned long n_wgs,
                      unsigned long iters);

/* Extension (no counterpart in the reference, which runs three moearc_matvec_q and up to three
 * moearc_add calls for attn.qkv, moe.rs:1942-1959): projection i (0 q, 1 k, 2 v) writes
 * out[i][r] = sum_c W_i[r][c] x[c] + bias[i][r] for r < rows[i] (bias[i] may be null), one launch
 * per distinct weight type. Bit-identical to the reference's sequence. type_ids, out, w, bias and
 * rows are HOST arrays of 3. Refusals: null c/x/arrays or a null out[i]/w[i] with rows[i] > 0 ->
 * -1; those of moearc_matvec_q for each projection -> -2. */
int moearc_attn_qkv(moearc_ctx *c, const unsigned int *type_ids, float *const *out,
                    const void *const *w, const float *const *bias, const unsigned long *rows,
                    const float *x, unsigned long n_cols);

/* Extension (no counterpart in the reference, which runs one moearc_matvec_q per token): the
 * projections of a prompt chunk as one MFMA matrix product, y[t][r] = sum_c W[r][c] x[t][c]
 * (+ bias[r]) for t < n_tok, r < n_rows; x f32 [n_tok][n_cols], y f32 [n_tok][n_rows]. Weights
 * Q8_0 (8), F16 (1), Q4_K (12), Q5_K (13), Q6_K (14) or MXFP4 (39), W 2-byte aligned. x enters as an f16
 * hi + lo pair (to 2^-22 relative; each |x| must stay below 65504), quantised payloads as exact
 * f16 integers / E2M1 values, block scales (and K-quant mins, against f32 block sums of x) in f32:
 * results are within 2 (32 + n_cols/32 + 5) 2^-24 sum|w x| per element (the matvec bound plus the
 * matrix core's 32-wide block sums). MXFP4 exponents of 253 and above (where the reference's
 * per-element products overflow) are not reproduced. Refusals: null c/y/w/x -> -1; another type,
 * n_cols not a multiple of 32 or of the block, an odd W address, n_rows, n_tok >= 2^31 -> -2.
 * n_rows or n_tok zero -> 0. */
int moearc_matmul_q(moearc_ctx *c, unsigned int type_id, float *y, const void *w, const float *x,
                    const float *bias, unsigned long n_tok, unsigned long n_rows, unsigned long n_cols);

/* ---- the attention block over a prompt chunk ---------------------------------------------------
 * Extension (no counterpart in the reference, whose prefill runs the whole model one token at a
 * time, session.rs:378-381 and moe.rs:1856-1862): the attention half of one block for n_tok
 * consecutive tokens in one call, the sequence of moe.rs:1942-2071 after attn.norm --
 *   q, k, v = W_{q,k,v} x (+ biases)        (moearc_attn_qkv, per token)
 *   q, k    = NeoX RoPE at pos[t]           (moearc_rope; K fused with the append below)
 *   K, V    -> pages[page_ids[t]], slot slots[t], f16   (moearc_rope_kv_append_chunk)
 *   attn    = chunked prefill over keys [pos0 + t + 1 - n_swa | 0, pos0 + t + 1)   (moearc_attn_prefill;
 *             a single token: moearc_attn_decode with its f32 q, the engine's own decode call)
 *   h      += W_o attn (+ bias_o)           (as moearc_attn_out, the residual add in the store)
 * with every earlier token's K/V already in the pages. n_tok = 1 is one decode step. All pointers
 * are device memory except `b` itself. With two or more tokens, projections whose weights
 * moearc_matmul_q takes run as one MFMA product each; the others token by token through the
 * batched matvec (up to 32 matrix-vector products per launch). */
typedef struct moearc_attn_block {
    unsigned int w_type[4];      /* GGUF type ids of W_q, W_k, W_v, W_o */
    const void *w[4];            /* W_q [n_head*head_dim][n_embd], W_k / W_v [n_head_kv*head_dim][n_embd],
                                    W_o [n_embd][n_head*head_dim] */
    const float *bias[4];        /* the matching biases, each may be NULL */
    const float *sinks;          /* [n_head] or NULL */
    void *k_pages, *v_pages;     /* f16 paged cache of this block */
    const unsigned int *block_table; /* the sequence's pages (a windowed block: its ring table) */
    unsigned long n_embd, n_head, n_head_kv, head_dim, page_tokens;
    unsigned long n_swa;         /* 0: full attention */
    unsigned long ring_pages;    /* a windowed block read through a ring table: the ring's pages, so the
                                    chunk is refused unless its keys fit (n_tok + n_swa - 1 <=
                                    ring_pages * page_tokens: later tokens of a chunk would otherwise
                                    overwrite keys earlier rows still attend to); 0: not a ring */
    float scale;                 /* attention scale, 1/sqrt(head_dim) */
    unsigned long n_rot;         /* rotated dimensions */
    float freq_base, freq_scale, ext_factor, attn_factor, corr_lo, corr_hi;  /* as moearc_rope */
} moearc_attn_block;

/* h f32 [n_tok][n_embd] (updated in place), x f32 [n_tok][n_embd] (attn.norm's output), pos i32,
 * page_ids / slots u32 [n_tok] (the tokens' cache places, as moearc_kv_pool_append_chunk returns
 * them), tokens at positions pos0 .. pos0 + n_tok - 1. Working memory is the context's (grown on
 * demand, kept). Refusals: null c, b, h, x, pos, page_ids or slots -> -1; a ring too small for the
 * chunk (see ring_pages) -> -2; then those of the calls above, in that order (nothing is enqueued
 * for a refusal found before the first launch). */
int moearc_attn_block_chunk(moearc_ctx *c, const moearc_attn_block *b, float *h, const float *x,
                            unsigned long n_tok, unsigned long pos0, const int *pos,
                            const unsigned int *page_ids, const unsigned int *slots);

/* Extension (no counterpart in the reference, which runs moearc_matvec_q, then moearc_add of the bias
 * and moearc_add into the residual for attn.proj, moe.rs:2063-2071): h[r] += W[r] . attn (+ bias[r])
 * for r < n_rows in one launch, bit-identical to that sequence. Refusals: null c/h/w/attn -> -1;
 * those of moearc_matvec_q -> -2. */
int moearc_attn_out(moearc_ctx *c, unsigned int type_id, float *h, const void *w, const float *bias,
                    const float *attn, unsigned long n_rows, unsigned long n_cols);

/* The stream the context enqueues on (a hipStream_t), so a caller can order its own work. */
void *moearc_ctx_stream(moearc_ctx *c);

#ifdef __cplusplus
}
#endif

#endif /* MOEARC_ATTN_H */
