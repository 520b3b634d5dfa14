/*
 * moearc_oracle.c -- CPU restatement of MoEArc's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the HIP path is compared against. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the product library
 * (moearc_amd) never links, imports or calls it, and must fail loudly when its own HIP build is
 * missing rather than fall back to this.
 *
 * Every function restates a reference function, cited as path:line relative to the reference
 * repository (chrisdesrochers/MoEArc). The arithmetic follows the reference's CPU twin
 * (crates/moearc-kernels/src/reference.rs): f64 accumulation, two passes (materialise the scores,
 * take the maximum, exponentiate, divide), sequential over heads. The one addition is the
 * attention sink, which reference.rs does not model and kernels.cpp:1864-1880 defines.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   orc_f16_to_f32 / orc_f32_to_f16  -- exhaustively against numpy's IEEE binary16 conversion
 *                                       (all 65,536 patterns, plus ties, subnormals, overflow);
 *   orc_attn_decode (no sink)        -- against torch's float64 scaled_dot_product_attention on a
 *                                       contiguous gather, plus the reference tests' closed forms
 *                                       (one key => V, one-key window => V, |out| <= max|V|);
 *   orc_attn_decode (sink)           -- against float64 SDPA with an extra zero-valued key whose
 *                                       additive bias is the sink, plus closed forms (one key =>
 *                                       V*sigmoid(s - sink); identical keys => mean(V)*n/(n+e^(sink-s));
 *                                       sink -> -1e30 equals no sink);
 *   orc_attn_prefill                 -- brute force: every row equals an independent float64
 *                                       masked softmax over the whole chunk;
 *   orc_kv_append / orc_kv_index     -- the reference test's exact-slot check (poisoned pool,
 *                                       neighbours untouched) and a numpy fancy-index gather;
 *   SplitMix64                       -- the published test vectors of the generator;
 *   orc_rope / orc_rope_yarn         -- complex multiplication by e^(i theta) in numpy complex128
 *                                       with the pairing built by slicing (halves for NeoX,
 *                                       even/odd for the adjacent convention); position 0 is the
 *                                       identity; rotated pairs keep their length times mscale;
 *                                       YaRN's ramp endpoints (pure extrapolation below corr_lo,
 *                                       freq_scale-interpolated above corr_hi); YaRN off equals
 *                                       plain RoPE;
 *   orc_dequant (all seven formats)  -- encoders written from the packing side of each format
 *                                       round-trip through it (Q4_K/Q5_K/Q6_K bit layouts and
 *                                       6-bit scale split); Q8_0 with d = 1 is its payload; MXFP4 is
 *                                       the OCP E2M1 code points times 2^(e-127), every byte value;
 *   orc_matvec_q                     -- numpy's float64 product of the decoded matrix.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_KV_F32 0u
#define ORC_KV_F16 1u

/* ---- RNG: crates/moearc-kernels/tests/common/mod.rs:11-37 ---------------------------- */

/* One SplitMix64 step (tests/common/mod.rs:19-25). */
uint64_t orc_splitmix64_next(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ull;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* `Rng::unit` (tests/common/mod.rs:31-33): uniform in [-1, 1), evaluated in f32. */
float orc_rng_unit(uint64_t *state) {
    uint32_t lo = (uint32_t) orc_splitmix64_next(state);
    float u = (float) lo / 4294967296.0f;
    return u * 2.0f - 1.0f;
}

void orc_rng_fill_unit(uint64_t *state, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_rng_unit(state);
}

/* ---- f16 codecs: reference.rs:123-149 (widen) and reference.rs:647-691 (narrow) ------- */

/* Binary16 -> binary32, lossless, subnormals renormalised (reference.rs:123-149). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            /* value = m * 2^-24; shift the leading one up to bit 10 */
            int shifts = 0;
            while ((m & 0x400u) == 0) { m <<= 1; ++shifts; }
            m &= 0x3FFu;
            bits = sign | ((uint32_t) (113 - shifts) << 23) | (m << 13);
        }
    } else if (e == 0x1F) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Binary32 -> binary16, IEEE round-to-nearest-even; overflow saturates to +-inf, subnormals are
 * rounded (not flushed), NaN stays NaN with payload 0x200 | mant>>13 (reference.rs:647-691). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t e32 = (x >> 23) & 0xFFu;
    uint32_t mant = x & 0x7FFFFFu;
    if (e32 == 0xFFu) return (uint16_t) (sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    int e = (int) e32 - 112; /* rebias 127 -> 15 */
    if (e >= 31) return (uint16_t) (sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t) sign;
        uint32_t full = mant | 0x800000u;
        int sh = 14 - e;
        uint32_t q = full >> sh;
        uint32_t rem = full & ((1u << sh) - 1u);
        uint32_t halfway = 1u << (sh - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q += 1u; /* carry may reach the normal range: correct */
        return (uint16_t) (sign | q);
    }
    uint32_t q = mant >> 13;
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) {
        q += 1u;
        if (q == 0x400u) {
            q = 0;
            e += 1;
            if (e >= 31) return (uint16_t) (sign | 0x7C00u);
        }
    }
    return (uint16_t) (sign | ((uint32_t) e << 10) | q);
}

void orc_f32_to_f16_n(const float *src, uint16_t *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_n(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

/* `KvType::store` (reference.rs:754-759): the value that lands in the cache. */
float orc_kv_store_value(float v, uint32_t kv_type) {
    return kv_type == ORC_KV_F16 ? orc_f16_to_f32(orc_f32_to_f16(v)) : v;
}

/* ---- KV layout: reference.rs:767-777 (kv_index), :781-802 (kv_append) ---------------- */

/* Element index of channel d of kv head `head` at (page, slot): layout [page][slot][kv_head][head_dim]. */
size_t orc_kv_index(uint32_t page, uint32_t slot, size_t head, size_t d, size_t n_kv_heads,
                    size_t head_dim, size_t page_tokens) {
    return (((size_t) page * page_tokens + slot) * n_kv_heads + head) * head_dim + d;
}

/* Host mirror of the append (reference.rs:781-802): pools hold f32 values (already rounded
 * through f16 when kv_type is F16). */
void orc_kv_append(float *k_pages, float *v_pages, const float *k, const float *v, uint32_t page,
                   uint32_t slot, size_t n_kv_heads, size_t head_dim, size_t page_tokens,
                   uint32_t kv_type) {
    for (size_t h = 0; h < n_kv_heads; ++h)
        for (size_t d = 0; d < head_dim; ++d) {
            size_t i = orc_kv_index(page, slot, h, d, n_kv_heads, head_dim, page_tokens);
            k_pages[i] = orc_kv_store_value(k[h * head_dim + d], kv_type);
            v_pages[i] = orc_kv_store_value(v[h * head_dim + d], kv_type);
        }
}

/* Device-format append: the pools hold the stored bytes (f32 or f16 bits), which is what the
 * kernel writes (kernels.cpp:1782-1799 with kv_store at :434-440). */
void orc_kv_append_raw(void *k_pages, void *v_pages, const float *k, const float *v, uint32_t page,
                       uint32_t slot, size_t n_kv_heads, size_t head_dim, size_t page_tokens,
                       uint32_t kv_type) {
    size_t n = n_kv_heads * head_dim;
    size_t base = ((size_t) page * page_tokens + slot) * n;
    for (size_t i = 0; i < n; ++i) {
        if (kv_type == ORC_KV_F16) {
            ((uint16_t *) k_pages)[base + i] = orc_f32_to_f16(k[i]);
            ((uint16_t *) v_pages)[base + i] = orc_f32_to_f16(v[i]);
        } else {
            ((float *) k_pages)[base + i] = k[i];
            ((float *) v_pages)[base + i] = v[i];
        }
    }
}

/* `kv_load` (kernels.cpp:427-432): one stored element as f32. */
static inline double kv_elem(const void *pages, size_t i, uint32_t kv_type) {
    if (kv_type == ORC_KV_F16) return (double) orc_f16_to_f32(((const uint16_t *) pages)[i]);
    return (double) ((const float *) pages)[i];
}

/* ---- attention: reference.rs:821-873 plus the sink of kernels.cpp:1864-1880 ----------- */

/* One query head over the span [kv_begin, n_kv), f64, two-pass. `scores` is caller scratch of
 * at least n_kv - kv_begin doubles. */
static void attend_head(double *out_d, const float *qh, const void *k_pages, const void *v_pages,
                        const uint32_t *block_table, const float *sink, size_t kvh,
                        size_t n_kv_heads, size_t head_dim, size_t kv_begin, size_t n_kv,
                        size_t page_tokens, float scale, uint32_t kv_type, double *scores) {
    size_t n = n_kv - kv_begin;
    double mx = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        size_t j = kv_begin + i;
        size_t base = orc_kv_index(block_table[j / page_tokens], (uint32_t) (j % page_tokens), kvh, 0,
                                   n_kv_heads, head_dim, page_tokens);
        double dot = 0.0;
        for (size_t d = 0; d < head_dim; ++d) dot += (double) qh[d] * kv_elem(k_pages, base + d, kv_type);
        scores[i] = dot * (double) scale;
        if (scores[i] > mx) mx = scores[i];
    }
    /* The sink is one more logit in the denominator with no value row; raw, compared against the
     * already-scaled scores (kernels.cpp:1864-1880). */
    if (sink && (double) *sink > mx) mx = (double) *sink;
    double denom = 0.0;
    for (size_t i = 0; i < n; ++i) {
        scores[i] = exp(scores[i] - mx);
        denom += scores[i];
    }
    if (sink) denom += exp((double) *sink - mx);
    for (size_t d = 0; d < head_dim; ++d) out_d[d] = 0.0;
    for (size_t i = 0; i < n; ++i) {
        size_t j = kv_begin + i;
        size_t base = orc_kv_index(block_table[j / page_tokens], (uint32_t) (j % page_tokens), kvh, 0,
                                   n_kv_heads, head_dim, page_tokens);
        for (size_t d = 0; d < head_dim; ++d) out_d[d] += scores[i] * kv_elem(v_pages, base + d, kv_type);
    }
    for (size_t d = 0; d < head_dim; ++d) out_d[d] /= denom;
}

/* Returns 0, or -2 for the arguments the reference refuses (kernels.cpp:1842-1852). Output in
 * f64 (`out_d`, may be NULL) and/or f32 (`out`, may be NULL), [n_heads][head_dim]. */
int orc_attn_decode(float *out, double *out_d, const float *q, const void *k_pages,
                    const void *v_pages, const uint32_t *block_table, const float *sinks,
                    size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t kv_begin, size_t n_kv,
                    size_t page_tokens, float scale, uint32_t kv_type, double *scratch) {
    if (kv_type != ORC_KV_F32 && kv_type != ORC_KV_F16) return -2;
    if (!n_heads || !n_kv_heads || !head_dim || !n_kv || !page_tokens) return -2;
    if (n_heads % n_kv_heads) return -2;
    if (kv_begin >= n_kv) return -2;
    size_t group = n_heads / n_kv_heads;
    double row[1024];
    if (head_dim > 1024) return -2;
    for (size_t h = 0; h < n_heads; ++h) {
        attend_head(row, q + h * head_dim, k_pages, v_pages, block_table, sinks ? sinks + h : NULL,
                    h / group, n_kv_heads, head_dim, kv_begin, n_kv, page_tokens, scale, kv_type,
                    scratch);
        for (size_t d = 0; d < head_dim; ++d) {
            if (out) out[h * head_dim + d] = (float) row[d];
            if (out_d) out_d[h * head_dim + d] = row[d];
        }
    }
    return 0;
}

/* Batched decode: sequence b uses block-table row b (stride bt_stride), span
 * [kv_begin[b], n_kv[b]) and query/output rows b. Equal to n_seqs independent decode calls. When
 * n_threads > 1 (and the file is built with OpenMP) the (sequence, head) pairs run in parallel;
 * the arithmetic of each pair is unchanged. `scratch` must hold n_threads * max_span doubles. */
int orc_attn_decode_batched(float *out, const float *q, const void *k_pages, const void *v_pages,
                            const uint32_t *block_tables, size_t bt_stride,
                            const uint32_t *kv_begin, const uint32_t *n_kv, const float *sinks,
                            size_t n_seqs, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                            size_t page_tokens, float scale, uint32_t kv_type, double *scratch,
                            size_t max_span, int n_threads) {
    if (kv_type != ORC_KV_F32 && kv_type != ORC_KV_F16) return -2;
    if (!n_heads || !n_kv_heads || !head_dim || !page_tokens || head_dim > 1024) return -2;
    if (n_heads % n_kv_heads) return -2;
    for (size_t b = 0; b < n_seqs; ++b) {
        if (kv_begin[b] >= n_kv[b]) return -2;
        if (n_kv[b] - kv_begin[b] > max_span) return -2;
    }
    size_t group = n_heads / n_kv_heads;
    long total = (long) (n_seqs * n_heads);
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1)
#endif
    for (long w = 0; w < total; ++w) {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        size_t b = (size_t) w / n_heads, h = (size_t) w % n_heads;
        double row[1024];
        attend_head(row, q + (b * n_heads + h) * head_dim, k_pages, v_pages,
                    block_tables + b * bt_stride, sinks ? sinks + h : NULL, h / group, n_kv_heads,
                    head_dim, kv_begin[b], n_kv[b], page_tokens, scale, kv_type,
                    scratch + (size_t) tid * max_span);
        for (size_t d = 0; d < head_dim; ++d) out[(b * n_heads + h) * head_dim + d] = (float) row[d];
    }
    (void) n_threads;
    return 0;
}

/* Prefill as the reference engine runs it (moe.rs:1856-1862, session.rs:378-381): query row i
 * sits at absolute position p = pos0 + i and is one decode call at n_kv = p + 1 with its own K/V
 * already in the cache; on a windowed layer (n_swa > 0) the span starts at max(0, p + 1 - n_swa)
 * (moe.rs:2020-2027), otherwise at 0. Only rows in [row_begin, row_end) are computed (a
 * subsample for large chunks); q and out are [n_q][n_heads][head_dim]. */
int orc_attn_prefill(float *out, const float *q, const void *k_pages, const void *v_pages,
                     const uint32_t *block_table, const float *sinks, size_t n_q, size_t pos0,
                     size_t n_swa, size_t row_begin, size_t row_end, size_t row_step,
                     size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t page_tokens,
                     float scale, uint32_t kv_type, double *scratch, int n_threads) {
    if (row_end > n_q) row_end = n_q;
    if (row_step == 0) row_step = 1;
    long rows = (long) ((row_end > row_begin) ? (row_end - row_begin + row_step - 1) / row_step : 0);
    size_t max_span = pos0 + n_q;
    int rc_any = 0;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1)
#endif
    for (long r = 0; r < rows; ++r) {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        size_t i = row_begin + (size_t) r * row_step;
        size_t nkv = pos0 + i + 1;
        size_t begin = (n_swa > 0 && nkv > n_swa) ? nkv - n_swa : 0;
        int rc = orc_attn_decode(out + i * n_heads * head_dim, NULL, q + i * n_heads * head_dim,
                                 k_pages, v_pages, block_table, sinks, n_heads, n_kv_heads, head_dim,
                                 begin, nkv, page_tokens, scale, kv_type,
                                 scratch + (size_t) tid * max_span);
        if (rc) rc_any = rc;
    }
    (void) n_threads;
    return rc_any;
}

/* ---- RoPE: reference.rs:468-505 (CPU twin) and kernels.cpp:1399-1468 (the kernel) -------- */

/* Channels of pair p: NeoX (p, p + n_dims/2), else (2p, 2p + 1) (reference.rs:451-457). */
static void rope_pair(size_t p, size_t n_dims, int neox, size_t *lo, size_t *hi) {
    *lo = neox ? p : 2 * p;
    *hi = neox ? p + n_dims / 2 : 2 * p + 1;
}

/* reference::rope: the angle table built per token by repeated f32 multiplication, as ggml's CPU
 * path does (theta *= theta_scale), f32 cos/sin, f32 rotation; channels >= n_dims copied. */
void orc_rope(float *out, const float *src, const int32_t *pos, size_t n_tokens, size_t n_heads,
              size_t head_dim, size_t n_dims, float freq_base, int neox) {
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    memcpy(out, src, n_tokens * n_heads * head_dim * sizeof(float));
    for (size_t t = 0; t < n_tokens; ++t) {
        float theta = (float) pos[t];
        for (size_t p = 0; p < n_dims / 2; ++p) {
            const float ct = cosf(theta), st = sinf(theta);
            for (size_t h = 0; h < n_heads; ++h) {
                const size_t base = (t * n_heads + h) * head_dim;
                size_t lo, hi;
                rope_pair(p, n_dims, neox, &lo, &hi);
                const float x0 = src[base + lo], x1 = src[base + hi];
                out[base + lo] = x0 * ct - x1 * st;
                out[base + hi] = x0 * st + x1 * ct;
            }
            theta *= theta_scale;
        }
    }
}

/* The kernel's closed form (kernels.cpp:1441-1466, ggml's rope_yarn), evaluated in f64 from the
 * f32 parameters (theta_scale rounded to f32 as the host computes it, kernels.cpp:1406): the
 * ground truth a f32 device implementation is compared to. out_d is f64. */
void orc_rope_yarn(double *out_d, const float *src, const int32_t *pos, size_t n_tokens,
                   size_t n_heads, size_t head_dim, size_t n_dims, float freq_base, float freq_scale,
                   float ext_factor, float attn_factor, float corr_lo, float corr_hi, int neox) {
    const double theta_scale = (double) powf(freq_base, -2.0f / (float) n_dims);
    for (size_t i = 0; i < n_tokens * n_heads * head_dim; ++i) out_d[i] = (double) src[i];
    for (size_t t = 0; t < n_tokens; ++t)
        for (size_t p = 0; p < n_dims / 2; ++p) {
            const double theta_extrap = (double) pos[t] * pow(theta_scale, (double) p);
            double theta = (double) freq_scale * theta_extrap;
            double mscale = (double) attn_factor;
            if (ext_factor != 0.0f) {
                const double y = ((double) p - corr_lo) / fmax(0.001, (double) corr_hi - corr_lo);
                const double ramp_mix = (1.0 - fmin(1.0, fmax(0.0, y))) * ext_factor;
                theta = theta * (1.0 - ramp_mix) + theta_extrap * ramp_mix;
                mscale *= 1.0 + 0.1 * log(1.0 / (double) freq_scale);
            }
            const double ct = cos(theta) * mscale, st = sin(theta) * mscale;
            for (size_t h = 0; h < n_heads; ++h) {
                const size_t base = (t * n_heads + h) * head_dim;
                size_t lo, hi;
                rope_pair(p, n_dims, neox, &lo, &hi);
                const double x0 = src[base + lo], x1 = src[base + hi];
                out_d[base + lo] = x0 * ct - x1 * st;
                out_d[base + hi] = x0 * st + x1 * ct;
            }
        }
}

/* The engine's per-token sequence (moe.rs:1987-2042): K rotated (closed form, rounded to f32),
 * then K and V appended at (page_ids[t], slots[t]) as moearc_kv_append stores them. */
void orc_rope_kv_append_chunk(void *k_pages, void *v_pages, const float *k, const float *v,
                              const int32_t *pos, const uint32_t *page_ids, const uint32_t *slots,
                              size_t n_tok, size_t n_kv_heads, size_t head_dim, size_t page_tokens,
                              size_t n_dims, float freq_base, float freq_scale, float ext_factor,
                              float attn_factor, float corr_lo, float corr_hi, int neox,
                              uint32_t kv_type, double *scratch_d, float *scratch_f) {
    const size_t row = n_kv_heads * head_dim;
    for (size_t t = 0; t < n_tok; ++t) {
        orc_rope_yarn(scratch_d, k + t * row, pos + t, 1, n_kv_heads, head_dim, n_dims, freq_base,
                      freq_scale, ext_factor, attn_factor, corr_lo, corr_hi, neox);
        for (size_t i = 0; i < row; ++i) scratch_f[i] = (float) scratch_d[i];
        if (slots[t] < page_tokens)
            orc_kv_append_raw(k_pages, v_pages, scratch_f, v + t * row, page_ids[t], slots[t],
                              n_kv_heads, head_dim, page_tokens, kv_type);
    }
}

/* ---- GGUF block formats and the matrix-vector product --------------------------------------
 * Restating reference.rs:42-336, which itself restates ggml's dequantize_row_* (ggml-quants.c,
 * a dependency of the reference not vendored in it). Values are expanded in f32 exactly as those
 * functions compute them (each product and difference rounded to f32, no contraction -- the
 * Makefile builds with -ffp-contract=off), then the products are accumulated in f64. */

#define ORC_TY_F32 0u
#define ORC_TY_F16 1u
#define ORC_TY_Q8_0 8u
#define ORC_TY_Q4_K 12u
#define ORC_TY_Q5_K 13u
#define ORC_TY_Q6_K 14u
#define ORC_TY_MXFP4 39u

/* Bytes and elements per block (reference.rs:79-104). 0 for an unknown type. */
size_t orc_block_bytes(uint32_t ty) {
    switch (ty) {
        case ORC_TY_F32: return 4;
        case ORC_TY_F16: return 2;
        case ORC_TY_Q8_0: return 34;
        case ORC_TY_Q4_K: return 144;
        case ORC_TY_Q5_K: return 176;
        case ORC_TY_Q6_K: return 210;
        case ORC_TY_MXFP4: return 17;
        default: return 0;
    }
}

size_t orc_block_elems(uint32_t ty) {
    switch (ty) {
        case ORC_TY_F32: case ORC_TY_F16: return 1;
        case ORC_TY_Q8_0: case ORC_TY_MXFP4: return 32;
        case ORC_TY_Q4_K: case ORC_TY_Q5_K: case ORC_TY_Q6_K: return 256;
        default: return 0;
    }
}

static float ld_f16(const uint8_t *p) { return orc_f16_to_f32((uint16_t) (p[0] | (p[1] << 8))); }

/* 2^(x - 128) (reference.rs:66-70): half the E8M0 value, to match the doubled E2M1 table. */
float orc_e8m0_half(uint8_t x) {
    const uint32_t bits = x < 2 ? 0x00200000u << x : ((uint32_t) x - 1u) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* The E2M1 code points doubled (reference.rs:52-55): magnitude codes 0..7 are 0, 0.5, 1, 1.5, 2,
 * 3, 4, 6 in the OCP MX format; bit 3 is the sign. */
static int mxfp4_doubled(unsigned code) {
    static const int mag[8] = {0, 1, 2, 3, 4, 6, 8, 12};
    return (code & 8u) ? -mag[code & 7u] : mag[code & 7u];
}

/* Sub-block j's 6-bit scale and min from the 12 packed bytes (reference.rs:150-160). */
static void scale_min_k4(const uint8_t *q, int j, unsigned *sc, unsigned *m) {
    if (j < 4) {
        *sc = q[j] & 63u;
        *m = q[j + 4] & 63u;
    } else {
        *sc = (q[j + 4] & 0xFu) | ((unsigned) (q[j - 4] >> 6) << 4);
        *m = (unsigned) (q[j + 4] >> 4) | ((unsigned) (q[j] >> 6) << 4);
    }
}

static void dq_block(uint32_t ty, const uint8_t *b, float *y) {
    switch (ty) {
        case ORC_TY_F32: memcpy(y, b, 4); break;
        case ORC_TY_F16: y[0] = ld_f16(b); break;
        case ORC_TY_Q8_0: { /* reference.rs:194-200: y = q * d */
            const float d = ld_f16(b);
            for (int j = 0; j < 32; ++j) y[j] = (float) (int8_t) b[2 + j] * d;
            break;
        }
        case ORC_TY_MXFP4: { /* reference.rs:202-217: byte j -> elements j (low), j + 16 (high) */
            const float d = orc_e8m0_half(b[0]);
            for (int j = 0; j < 16; ++j) {
                y[j] = (float) mxfp4_doubled(b[1 + j] & 0xFu) * d;
                y[j + 16] = (float) mxfp4_doubled(b[1 + j] >> 4) * d;
            }
            break;
        }
        case ORC_TY_Q4_K: { /* reference.rs:219-244 */
            const float d = ld_f16(b), dmin = ld_f16(b + 2);
            const uint8_t *sc = b + 4, *qs = b + 16;
            for (int g = 0; g < 4; ++g) {  /* 64 elements: low nibbles, then high, of 32 bytes */
                unsigned s0, m0, s1, m1;
                scale_min_k4(sc, 2 * g, &s0, &m0);
                scale_min_k4(sc, 2 * g + 1, &s1, &m1);
                const float d0 = d * (float) s0, n0 = dmin * (float) m0;
                const float d1 = d * (float) s1, n1 = dmin * (float) m1;
                for (int l = 0; l < 32; ++l) {
                    const float lo = d0 * (float) (qs[32 * g + l] & 0xF);
                    const float hi = d1 * (float) (qs[32 * g + l] >> 4);
                    y[64 * g + l] = lo - n0;
                    y[64 * g + 32 + l] = hi - n1;
                }
            }
            break;
        }
        case ORC_TY_Q5_K: { /* reference.rs:246-277: fifth bits in qh, bit 2g (low) / 2g+1 (high) */
            const float d = ld_f16(b), dmin = ld_f16(b + 2);
            const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
            for (int g = 0; g < 4; ++g) {
                unsigned s0, m0, s1, m1;
                scale_min_k4(sc, 2 * g, &s0, &m0);
                scale_min_k4(sc, 2 * g + 1, &s1, &m1);
                const float d0 = d * (float) s0, n0 = dmin * (float) m0;
                const float d1 = d * (float) s1, n1 = dmin * (float) m1;
                for (int l = 0; l < 32; ++l) {
                    const unsigned ql = qs[32 * g + l];
                    const unsigned q0 = (ql & 0xFu) + ((qh[l] >> (2 * g)) & 1u) * 16u;
                    const unsigned q1 = (ql >> 4) + ((qh[l] >> (2 * g + 1)) & 1u) * 16u;
                    const float lo = d0 * (float) q0, hi = d1 * (float) q1;
                    y[64 * g + l] = lo - n0;
                    y[64 * g + 32 + l] = hi - n1;
                }
            }
            break;
        }
        case ORC_TY_Q6_K: { /* reference.rs:279-303 */
            const float d = ld_f16(b + 208);
            for (int n = 0; n < 2; ++n) {
                const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
                const int8_t *sc = (const int8_t *) (b + 192 + 8 * n);
                for (int l = 0; l < 32; ++l) {
                    const int is = l / 16;
                    const int q[4] = {
                        (int) ((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32,
                        (int) ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32,
                        (int) ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32,
                        (int) ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32};
                    for (int c = 0; c < 4; ++c) {
                        const float ds = d * (float) sc[is + 2 * c];
                        y[128 * n + 32 * c + l] = ds * (float) q[c];
                    }
                }
            }
            break;
        }
    }
}

/* Expand nblocks blocks (reference.rs:168-192). -2 for an unknown type. */
int orc_dequant(uint32_t ty, const uint8_t *src, size_t nblocks, float *dst) {
    const size_t bb = orc_block_bytes(ty), be = orc_block_elems(ty);
    if (!bb) return -2;
    for (size_t i = 0; i < nblocks; ++i) dq_block(ty, src + i * bb, dst + i * be);
    return 0;
}

/* out[r] = sum_c W[r][c] x[c], W dequantised to f32 then accumulated in f64 (reference.rs:305-336).
 * absum (nullable) receives sum_c |W[r][c] x[c]| per row, the scale of the reference tests'
 * tolerance (kernels_gpu.rs:126-137). -2 for an unknown type or a ragged row. */
int orc_matvec_q(uint32_t ty, const uint8_t *w, const float *x, size_t n_rows, size_t n_cols,
                 float *out, double *absum, int n_threads) {
    const size_t bb = orc_block_bytes(ty), be = orc_block_elems(ty);
    if (!bb || n_cols % be) return -2;
    const size_t nb = n_cols / be;
    int rc = 0;
#ifdef _OPENMP
#pragma omp parallel for num_threads(n_threads > 0 ? n_threads : 1) schedule(static)
#endif
    for (size_t r = 0; r < n_rows; ++r) {
        float row[256];
        double acc = 0.0, mag = 0.0;
        for (size_t i = 0; i < nb; ++i) {
            dq_block(ty, w + (r * nb + i) * bb, row);
            for (size_t j = 0; j < be; ++j) {
                const double p = (double) row[j] * (double) x[i * be + j];
                acc += p;
                mag += fabs(p);
            }
        }
        out[r] = (float) acc;
        if (absum) absum[r] = mag;
    }
    (void) n_threads;
    return rc;
}
