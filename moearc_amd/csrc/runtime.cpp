// Host side of libmoearc_attn.so: the C ABI declared in include/moearc_attn.h.
//
// A context owns one HIP stream and the kernels' code object (moearc_attn_gfx950.co, beside this
// library), loaded with hipModuleLoad; every entry point validates its arguments on the host, in
// the reference's order, before anything is enqueued, then launches with hipModuleLaunchKernel
// on the context's stream and returns without waiting (the reference's "0 = accepted" contract,
// kernels.cpp:875-880).
//
// Built with the host compiler against the HIP runtime API only; no device code lives here.
#include "moearc_attn.h"

#include <cmath>
#include <cstddef>

#include <hip/hip_runtime_api.h>

#include <dlfcn.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "launch_args.h"

namespace {

constexpr int OK = 0;
constexpr int ERR = -1;
constexpr int ERR_ARG = -2;

struct Pending {
    std::string key;
    hipEvent_t start, stop;
};

struct KernelTime {
    std::string key;
    unsigned long long ns;
    unsigned long long calls;
};

std::string library_dir() {
    Dl_info info;
    if (dladdr((void *) &library_dir, &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        const size_t s = p.rfind('/');
        if (s != std::string::npos) return p.substr(0, s);
    }
    return ".";
}

bool is_pow2(unsigned long x) { return x && !(x & (x - 1)); }

// Matvec weight formats (GGUF type ids), their kernel-name stems and profiling key names.
constexpr uint32_t kMvTypes[7] = {0, 1, 8, 12, 13, 14, 39};
constexpr const char *kMvNames[7] = {"f32", "f16", "q8_0", "q4_k", "q5_k", "q6_k", "mxfp4"};
constexpr const char *kMvKeys[7] = {"F32", "F16", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "MXFP4"};

int mv_type_index(unsigned ty) {
    for (int t = 0; t < 7; ++t)
        if (kMvTypes[t] == ty) return t;
    return -1;
}

uint32_t log2u(unsigned long x) {
    uint32_t s = 0;
    while ((1ul << s) < x) ++s;
    return s;
}

}  // namespace

struct moearc_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipModule_t module = nullptr;
    hipFunction_t f_zero = nullptr, f_quant = nullptr, f_append = nullptr, f_append_chunk = nullptr;
    hipFunction_t f_rope = nullptr, f_rope_f16 = nullptr, f_rope_append_chunk = nullptr, f_rope_append64 = nullptr;
    hipFunction_t f_rope_qkv64 = nullptr;  // RoPE of q and the fused K/V append in one launch
    hipFunction_t f_rope_sums64 = nullptr;  // the same from the q/k/v product's split-K sums
    bool block_fused = true;  // MOEARC_BLOCK_FUSED=0: the attention block's fused steps as separate launches
    hipFunction_t f_dec_general = nullptr;
    hipFunction_t f_dec_fast[2] = {};  // split kernels (kDecodeVariants)
    hipFunction_t f_dec_merge = nullptr;
    unsigned merge_threads = 0;  // the merge kernel's launch bound (its work-group size)
    hipFunction_t f_mv[7][4] = {};  // matvec: format (F32 F16 Q8_0 Q4_K Q5_K Q6_K MXFP4) x pieces per lane 1/2/4/8
    hipFunction_t f_add = nullptr, f_read_floor = nullptr, f_mfma_floor = nullptr;
    hipFunction_t f_mm[6][2] = {}, f_split = nullptr, f_split8 = nullptr, f_bsums = nullptr;  // Q8_0 F16 Q4_K Q5_K MXFP4 Q6_K x 16 / 32 rows per wave
    hipFunction_t f_mm2[6] = {};  // Q8_0, F16, Q4_K, Q5_K, Q6_K, MXFP4: 128 x 128 tiles on the 32x32x16 MFMA
    hipFunction_t f_mm2w[3] = {};  // Q8_0, F16, MXFP4 on 128 tokens x 256 rows, eight waves
    uint16_t *mm_ws = nullptr;  // f16 hi / lo split of a chunk's activations
    size_t mm_ws_halves = 0;
    float *mm_part = nullptr;   // the k-slices' sums of split chunk products
    size_t mm_part_floats = 0;
    hipFunction_t f_mm_reduce = nullptr;
    hipFunction_t f_mm_reduce4 = nullptr;  // four elements per lane, when every address allows
    hipFunction_t f_prefill[4] = {};      // group 1, 2, 4, 8
    hipFunction_t f_prefill_precise[4] = {};  // the same with p split into f16 hi + lo
    bool prefill_precise = false;         // MOEARC_PREFILL_PRECISE=1: p split into f16 hi + lo
    bool profiling = false;        // MOEARC_PROFILE_EVENTS=1: one event bracket per tracked call
    bool profile_kernels = false;  // MOEARC_PROFILE_KERNELS=1: also every kernel inside a call
    int scope_depth = 0;           // > 0 while an entry point's own bracket is open
    // Errors found after a call returned 0, reported by the next moearc_sync: a device word the
    // chunk-append kernels set when a device-resident slot lies outside its page (err_armed: a
    // launch that can set it was enqueued since the last check), and a failed HIP call in an
    // entry point that returns nothing (moearc_free_device).
    uint32_t *err_word = nullptr;
    bool err_armed = false;
    bool deferred_error = false;
    // The code object's fixed record array (moearc_decode_scratch): its device address in this
    // context's module instance, read once at creation, and its size in floats.
    float *scratch = nullptr;
    size_t scratch_floats = 0;
    int quiet = 0;  // > 0 during an allocation-free call: no profiling events are taken
    std::vector<Pending> pending;
    std::vector<KernelTime> totals;
    std::vector<hipEvent_t> event_pool;
    // split-K workspace: the partial records of the split kernel (per query head and work item)
    float *ws = nullptr;
    size_t ws_floats = 0;
    int decode_variant_override = -1;  // MOEARC_DECODE_VARIANT, e.g. "4x2x4"
    unsigned long split_override = 0;  // MOEARC_DECODE_SPLIT (keys per split)
    float *blk_ws = nullptr;  // attention-block chunk: q, k, v, f16 q, attention output, projection
    size_t blk_ws_bytes = 0;
    unsigned long mv_rpw_override = 0;  // MOEARC_MATVEC_RPW: rows per wave of the matvec launches
    unsigned mv_waves_override = 0;     // MOEARC_MATVEC_WAVES: 4 or 8 waves per work-group
    unsigned n_cu = 0;       // compute units of the device
    // Prefill pair balance (PrefillArgs::boost_a, boost_b; MOEARC_PF_BOOST="a,b", "0,0" turns it
    // off). Measured on config 4: while two work-groups share a CU the older one's waves take ~65%
    // of the issue slots; with a = 1.41, b = 0.77 the younger keeps priority 1 for as long as makes
    // the two end together (loop ends 104.4 / 104.8 µs against 94.9 / 108.0 without).
    float pf_boost_a = 1.41f, pf_boost_b = 0.77f;
    int mm_wide = -1;  // MOEARC_MM_WIDE: the chunk product's wide tiles (0: never, 1: always, -1: by grid)
    int mm_split_wg = -1;  // MOEARC_MM_SPLIT_WG: work-groups per CU the chunk product's split-K aims at (0: none; -1: by chunk)
};

namespace {

hipEvent_t take_event(moearc_ctx *c) {
    if (!c->event_pool.empty()) {
        hipEvent_t e = c->event_pool.back();
        c->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void flush_events(moearc_ctx *c) {
    for (auto &p : c->pending) {
        float ms = 0.f;
        if (hipEventSynchronize(p.stop) == hipSuccess &&
            hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
            const unsigned long long ns = (unsigned long long) (ms * 1.0e6);
            bool found = false;
            for (auto &t : c->totals)
                if (t.key == p.key) {
                    t.ns += ns;
                    t.calls += 1;
                    found = true;
                    break;
                }
            if (!found) c->totals.push_back(KernelTime{p.key, ns, 1});
        }
        c->event_pool.push_back(p.start);
        c->event_pool.push_back(p.stop);
    }
    c->pending.clear();
}

void record_bracket(moearc_ctx *c, hipEvent_t start, const char *what, unsigned long r,
                    unsigned long m) {
    hipEvent_t e1 = take_event(c);
    if (!e1) {
        c->event_pool.push_back(start);
        return;
    }
    if (hipEventRecord(e1, c->stream) != hipSuccess) {
        c->event_pool.push_back(start);
        c->event_pool.push_back(e1);
        return;
    }
    char key[96];
    std::snprintf(key, sizeof(key), "%s r%lu m%lu", what, r, m);
    c->pending.push_back(Pending{key, start, e1});
    if (c->pending.size() >= 16384) flush_events(c);
}

// Whether a launch keyed `what` gets its own event bracket. Each tracked call is recorded once
// under one key, as the reference records each submission (kernels.cpp:1905-1916): a kernel
// launched inside a call that holds its own bracket (scope_depth > 0), or one whose entry point
// the reference does not track (what == nullptr), is recorded only with MOEARC_PROFILE_KERNELS=1,
// under "kernel <what>" -- consumers that sum every key then still count each call once.
bool tracks(const moearc_ctx *c, const char *what) {
    if (!c->profiling || c->quiet) return false;
    return c->profile_kernels || (what && c->scope_depth == 0);
}

// Launch `f` with one by-value argument block. With profiling on, a HIP event pair brackets the
// launch under the key "<what> r<r> m<m>" (the reference's key format, kernels.cpp:1905-1916).
template <typename Args>
int launch3d(moearc_ctx *c, hipFunction_t f, unsigned grid, unsigned grid_y, unsigned grid_z, unsigned block,
             const Args &args, const char *what, unsigned long r, unsigned long m,
             unsigned lds_bytes = 0, const char *kernel = nullptr) {
    if (!f) return ERR;
    hipEvent_t e0 = nullptr;
    const bool own = what && c->scope_depth == 0;  // this launch is the whole tracked call
    if (tracks(c, what) && (e0 = take_event(c))) {
        if (hipEventRecord(e0, c->stream) != hipSuccess) {
            c->event_pool.push_back(e0);
            e0 = nullptr;
        }
    }
    size_t size = sizeof(Args);
    void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, (void *) &args, HIP_LAUNCH_PARAM_BUFFER_SIZE,
                      &size, HIP_LAUNCH_PARAM_END};
    const hipError_t err =
        hipModuleLaunchKernel(f, grid, grid_y, grid_z, block, 1, 1, lds_bytes, c->stream, nullptr, config);
    if (e0) {
        if (own) {
            record_bracket(c, e0, what, r, m);
        } else {
            char k[80];
            std::snprintf(k, sizeof(k), "kernel %s", kernel ? kernel : (what ? what : "?"));
            record_bracket(c, e0, k, r, m);
        }
    }
    return err == hipSuccess ? OK : ERR;
}

template <typename Args>
int launch2d(moearc_ctx *c, hipFunction_t f, unsigned grid, unsigned grid_y, unsigned block,
             const Args &args, const char *what, unsigned long r, unsigned long m,
             unsigned lds_bytes = 0, const char *kernel = nullptr) {
    return launch3d(c, f, grid, grid_y, 1, block, args, what, r, m, lds_bytes, kernel);
}

template <typename Args>
int launch(moearc_ctx *c, hipFunction_t f, unsigned grid, unsigned block, const Args &args,
           const char *what, unsigned long r, unsigned long m, const char *kernel = nullptr) {
    return launch2d(c, f, grid, 1, block, args, what, r, m, 0, kernel);
}

int ensure_workspace(moearc_ctx *c, size_t floats) {
    if (floats <= c->ws_floats) return OK;
    if (c->ws) {
        // the previous workspace may still be read by queued launches
        if (hipStreamSynchronize(c->stream) != hipSuccess) return ERR;
        if (hipFree(c->ws) != hipSuccess) return ERR;
        c->ws = nullptr;
        c->ws_floats = 0;
    }
    if (hipMalloc((void **) &c->ws, floats * sizeof(float)) != hipSuccess) return ERR;
    c->ws_floats = floats;
    return OK;
}

// ---- decode dispatch ----------------------------------------------------------------------------

struct SeqSpan {
    uint32_t begin, end;
};

// The key spans of a decode call: the single call's (begin0, end0), or the batched call's host
// arrays. Read in place, so the dispatch allocates nothing on the host either.
struct SpanList {
    const unsigned int *kv_begin = nullptr, *n_kv = nullptr;
    uint32_t begin0 = 0, end0 = 0;
    size_t n = 0;
    SeqSpan at(size_t i) const { return kv_begin ? SeqSpan{kv_begin[i], n_kv[i]} : SeqSpan{begin0, end0}; }
};

// The split-K kernel masks keys with -inf scores before multiplying by scale*log2(e) and takes
// its running maximum on raw scores, so it needs a positive, finite scale; any other scale runs on
// the general kernel.
bool fast_decode_ok(unsigned long n_heads, unsigned long n_kv_heads, unsigned long head_dim,
                    unsigned long page_tokens, unsigned int kv_type, float scale) {
    return kv_type == 1u && head_dim == 64 && n_heads / n_kv_heads <= 16 && n_kv_heads <= 0xFFFFul &&
           is_pow2(page_tokens) && page_tokens <= (1ul << 30) && scale > 0.f && scale <= 3.0e38f;
}

// Split-K decode variants (moearc_attn_decode_f16d64_k<kb>w<wpk>t<tiles>): kb KV heads x wpk
// waves per work-group, each wave computing `tiles` 32-key tiles per chunk with all of their loads
// in flight; the work-group count the split length aims for.
struct DecodeVariant {
    const char *name;
    unsigned kb, wpk, tiles, target_wgs;
};
constexpr int kNumDecodeVariants = 2;
constexpr DecodeVariant kDecodeVariants[kNumDecodeVariants] = {
    {"4x2x4", 4, 2, 4, 256},  // 8 waves (2 per SIMD at 214 VGPRs): one work-group per CU
    {"1x4x1", 1, 4, 1, 1024}, // 4 waves, many small work-groups: short spans, windows
};

// Variant and keys per split. The long-span variant reads 512 contiguous bytes of every key row
// per work-group and keeps 32 KiB per wave in flight; it is used when the launch's keys give it
// at least ~3/4 of a work-group per CU at one chunk per wave (config 2's 32768 keys give exactly
// one), else the one-KV-head variant, which gives 8x the work-groups per key. The split length is
// the shortest whole number of chunks for which the launch has at most the variant's target
// work-group count (all resident at once: a second round of work-groups would start only as the
// first finishes and double the time); ragged spans make the count a step function of the length,
// hence the search.
void plan_split(const moearc_ctx *c, const SeqSpan *spans, size_t cnt, unsigned long G, int &variant,
                uint32_t &split_len) {
    uint64_t keys = 0, longest = 0;
    for (size_t i = 0; i < cnt; ++i) {
        keys += (uint64_t) (spans[i].end - spans[i].begin);
        longest = std::max<uint64_t>(longest, spans[i].end - spans[i].begin);
    }
    auto nkb_of = [&](int v) { return (G + kDecodeVariants[v].kb - 1) / kDecodeVariants[v].kb; };
    auto chunk_of = [&](int v) { return 32ull * kDecodeVariants[v].wpk * kDecodeVariants[v].tiles; };
    variant = keys * nkb_of(0) / chunk_of(0) >= 192 ? 0 : 1;
    if (c->decode_variant_override >= 0) variant = c->decode_variant_override;
    const uint64_t quantum = chunk_of(variant), nkb = nkb_of(variant);
    const uint64_t target = kDecodeVariants[variant].target_wgs;
    auto wgs_at = [&](uint64_t len) {
        uint64_t items = 0;
        for (size_t i = 0; i < cnt; ++i) items += (spans[i].end - spans[i].begin + len - 1) / len;
        return items * nkb;
    };
    uint64_t lo = 1, hi = std::max<uint64_t>(1, (longest + quantum - 1) / quantum);  // in chunks
    while (lo < hi) {
        const uint64_t mid = (lo + hi) / 2;
        if (wgs_at(mid * quantum) <= target) hi = mid;
        else lo = mid + 1;
    }
    uint64_t len = c->split_override ? c->split_override : lo * quantum;
    len = std::max<uint64_t>(len, quantum);
    len = (len + quantum - 1) / quantum * quantum;
    split_len = (uint32_t) std::min<uint64_t>(len, 0x40000000ull);
}

// Launch layouts. The leading scalars are the kernel's preloaded arguments (the code object is
// built with kernarg preloading of 14 dwords); the struct follows at its natural alignment, as the
// kernel's parameter list places it.
struct DecodeLaunch {
    const uint16_t *k_pages, *v_pages;
    const uint32_t *bt0;
    const float *q0;
    uint32_t kvb0, nkv0, slen0, next0;
    uint32_t geo0, geo1;
    DecodeArgs a;
};
struct MergeLaunch {
    const float *rec_o, *rec_ml;
    void *out;
    const float *sinks;
    uint32_t n_items, next0, n_heads, out_f16;
    MergeArgs m;
};
static_assert(offsetof(DecodeLaunch, a) == 56, "decode kernel argument layout");
static_assert(offsetof(MergeLaunch, m) == 48 && sizeof(MergeLaunch) == 48 + sizeof(MergeArgs),
              "merge kernel argument layout");
static_assert(sizeof(DecodeLaunch) == 56 + sizeof(DecodeArgs), "decode kernel argument layout");

// Where a decode call keeps its partial records: the context's workspace (grown on demand), or a
// fixed buffer of `cap` floats that the call must fit (the allocation-free entry point).
struct RecordSpace {
    float *fixed = nullptr;
    size_t cap = 0;
};

// The spans of launch group s0 (at most MOEARC_MAX_SEQS_PER_LAUNCH sequences) into sub[].
size_t group_spans(const SpanList &spans, size_t s0, SeqSpan *sub) {
    const size_t cnt = std::min<size_t>(MOEARC_MAX_SEQS_PER_LAUNCH, spans.n - s0);
    for (size_t i = 0; i < cnt; ++i) sub[i] = spans.at(s0 + i);
    return cnt;
}

// Work items (splits over all sequences) of a launch group under its plan.
uint64_t group_items(const SeqSpan *sub, size_t cnt, uint32_t split_len) {
    uint64_t items = 0;
    for (size_t i = 0; i < cnt; ++i) items += (sub[i].end - sub[i].begin + (uint64_t) split_len - 1) / split_len;
    return items;
}

int decode_launch_body(moearc_ctx *c, void *out, unsigned int out_f16, const float *q,
                       const void *k_pages, const void *v_pages, const unsigned int *block_tables,
                       unsigned long bt_stride, const SpanList &spans, const float *sinks,
                       unsigned long n_heads, unsigned long n_kv_heads, unsigned long head_dim,
                       unsigned long page_tokens, float scale, unsigned int kv_type, RecordSpace rs);

int decode_launch(moearc_ctx *c, void *out, unsigned int out_f16, const float *q,
                  const void *k_pages, const void *v_pages, const unsigned int *block_tables,
                  unsigned long bt_stride, const SpanList &spans, const float *sinks,
                  unsigned long n_heads, unsigned long n_kv_heads, unsigned long head_dim,
                  unsigned long page_tokens, float scale, unsigned int kv_type, RecordSpace rs = {}) {
    // A fixed record buffer must hold every launch group's records: checked for all groups before
    // anything is enqueued, so a refusal leaves the stream untouched.
    if (rs.fixed && fast_decode_ok(n_heads, n_kv_heads, head_dim, page_tokens, kv_type, scale)) {
        SeqSpan sub[MOEARC_MAX_SEQS_PER_LAUNCH];
        for (size_t s0 = 0; s0 < spans.n; s0 += MOEARC_MAX_SEQS_PER_LAUNCH) {
            const size_t cnt = group_spans(spans, s0, sub);
            int variant = 0;
            uint32_t split_len = 0;
            plan_split(c, sub, cnt, n_kv_heads, variant, split_len);
            const uint64_t items = group_items(sub, cnt, split_len);
            if (items > cnt && (uint64_t) n_heads * items * 66u > rs.cap) return ERR_ARG;
        }
    }
    // With profiling on, the whole call (split and merge launches, SWA and full layers alike) is
    // one bracket under the reference's key "attn_decode r<n_heads> m<head_dim>"
    // (kernels.cpp:1905-1916); its kernels are timed on their own only with
    // MOEARC_PROFILE_KERNELS=1. The allocation-free entry point records no events.
    hipEvent_t call0 = nullptr;
    if (!rs.fixed && tracks(c, "attn_decode") && (call0 = take_event(c))) {
        if (hipEventRecord(call0, c->stream) != hipSuccess) {
            c->event_pool.push_back(call0);
            call0 = nullptr;
        }
    }
    ++c->scope_depth;
    const int rc_all = decode_launch_body(c, out, out_f16, q, k_pages, v_pages, block_tables,
                                          bt_stride, spans, sinks, n_heads, n_kv_heads, head_dim,
                                          page_tokens, scale, kv_type, rs);
    --c->scope_depth;
    if (call0) record_bracket(c, call0, "attn_decode", n_heads, head_dim);
    return rc_all;
}

int decode_launch_body(moearc_ctx *c, void *out, unsigned int out_f16, const float *q,
                       const void *k_pages, const void *v_pages, const unsigned int *block_tables,
                       unsigned long bt_stride, const SpanList &spans, const float *sinks,
                       unsigned long n_heads, unsigned long n_kv_heads, unsigned long head_dim,
                       unsigned long page_tokens, float scale, unsigned int kv_type, RecordSpace rs) {
    const bool fast_shape = fast_decode_ok(n_heads, n_kv_heads, head_dim, page_tokens, kv_type, scale);
    SeqSpan sub[MOEARC_MAX_SEQS_PER_LAUNCH];
    for (size_t s0 = 0; s0 < spans.n; s0 += MOEARC_MAX_SEQS_PER_LAUNCH) {
        const size_t cnt = group_spans(spans, s0, sub);
        const float *qb = q + s0 * n_heads * head_dim;
        const size_t out_off = s0 * n_heads * head_dim * (out_f16 ? 2 : 4);
        void *ob = (char *) out + out_off;
        const unsigned int *btb = block_tables + s0 * bt_stride;
        int variant = 0;
        uint32_t split_len = 0;
        if (fast_shape) plan_split(c, sub, cnt, n_kv_heads, variant, split_len);
        if (!fast_shape) {
            DecodeGeneralArgs a{};
            a.q = qb;
            a.k_pages = k_pages;
            a.v_pages = v_pages;
            a.block_tables = btb;
            a.sinks = sinks;
            a.out = ob;
            a.bt_stride = bt_stride;
            a.n_heads = (uint32_t) n_heads;
            a.n_kv_heads = (uint32_t) n_kv_heads;
            a.head_dim = (uint32_t) head_dim;
            a.page_tokens = (uint32_t) page_tokens;
            a.kv_type = kv_type;
            a.out_f16 = out_f16;
            a.scale = scale;
            a.n_seqs = (uint32_t) cnt;
            for (size_t i = 0; i < cnt; ++i) {
                a.kv_begin[i] = sub[i].begin;
                a.n_kv[i] = sub[i].end;
            }
            const int rc = launch(c, c->f_dec_general, (unsigned) (cnt * n_heads), 256, a,
                                  "attn_decode.general", n_heads, head_dim);
            if (rc) return rc;
            continue;
        }
        const DecodeVariant &dv = kDecodeVariants[variant];
        const size_t nkb = (n_kv_heads + dv.kb - 1) / dv.kb;
        DecodeLaunch L{};
        DecodeArgs &a = L.a;
        a.q = qb;
        a.block_tables = btb;
        a.sinks = sinks;
        a.out = ob;
        a.bt_stride = bt_stride;
        a.out_f16 = out_f16;
        a.scale_log2e = scale * 1.4426950408889634f;
        a.n_seqs = (uint32_t) cnt;
        uint32_t items = 0;
        for (size_t i = 0; i < cnt; ++i) {
            a.item_begin[i] = items;
            a.kv_begin[i] = sub[i].begin;
            a.n_kv[i] = sub[i].end;
            a.split_len[i] = split_len;
            const uint64_t n_split = (sub[i].end - sub[i].begin + (uint64_t) split_len - 1) / split_len;
            if (items + n_split > 0x7FFFFFFFull) return ERR_ARG;
            items += (uint32_t) n_split;
        }
        for (size_t i = cnt; i <= MOEARC_MAX_SEQS_PER_LAUNCH; ++i) a.item_begin[i] = items;
        const size_t wgs = (size_t) items * nkb;
        if (wgs > 0x7FFFFFFFull) return ERR_ARG;
        const bool any_split = items > cnt;  // some sequence has more than one split
        if (any_split) {
            const size_t rec = (size_t) n_heads * items;
            float *ws = rs.fixed;
            if (ws) {
                if (rec * 66 > rs.cap) return ERR_ARG;  // checked for every group before the first launch
            } else {
                if (ensure_workspace(c, rec * 66)) return ERR;
                ws = c->ws;
            }
            a.rec_o = ws;
            a.rec_ml = ws + rec * 64;
        }
        a.n_items = items;
        L.k_pages = (const uint16_t *) k_pages;
        L.v_pages = (const uint16_t *) v_pages;
        L.bt0 = btb;
        L.q0 = qb;
        L.kvb0 = a.kv_begin[0];
        L.nkv0 = a.n_kv[0];
        L.slen0 = a.split_len[0];
        L.next0 = a.item_begin[1];
        L.geo0 = log2u(page_tokens) | (uint32_t) n_kv_heads << 16;
        L.geo1 = (uint32_t) nkb | (uint32_t) (n_heads / n_kv_heads) << 16;
        const int rc = launch(c, c->f_dec_fast[variant], (unsigned) wgs, 64u * dv.kb * dv.wpk, L,
                              "attn_decode.split", n_heads, head_dim);
        if (rc) return rc;
        if (any_split) {
            MergeLaunch M{};
            M.rec_o = a.rec_o;
            M.rec_ml = a.rec_ml;
            M.out = ob;
            M.sinks = sinks;
            M.n_items = items;
            M.next0 = a.item_begin[1];
            M.n_heads = (uint32_t) n_heads;
            M.out_f16 = out_f16;
            for (size_t i = 0; i <= MOEARC_MAX_SEQS_PER_LAUNCH; ++i) M.m.item_begin[i] = a.item_begin[i];
            M.m.item_begin[MOEARC_MAX_SEQS_PER_LAUNCH + 1] = items;
            const int rm = launch2d(c, c->f_dec_merge, (unsigned) n_heads, (unsigned) cnt, c->merge_threads,
                                    M, "attn_decode.merge", n_heads, head_dim);
            if (rm) return rm;
        }
    }
    return OK;
}

// Frees everything a (possibly half-built) context holds and returns nullptr. Teardown has no
// caller to report a failure to (moearc_ctx_destroy returns nothing, ffi.rs:21), so the results
// of these calls are deliberately dropped.
moearc_ctx *release(moearc_ctx *c) {
    if (c->stream) (void) hipStreamSynchronize(c->stream);
    for (auto &p : c->pending) {
        (void) hipEventDestroy(p.start);
        (void) hipEventDestroy(p.stop);
    }
    for (auto e : c->event_pool) (void) hipEventDestroy(e);
    for (void *p : {(void *) c->ws, (void *) c->blk_ws, (void *) c->mm_ws, (void *) c->mm_part,
                    (void *) c->err_word})
        if (p) (void) hipFree(p);
    if (c->module) (void) hipModuleUnload(c->module);
    if (c->stream) (void) hipStreamDestroy(c->stream);
    delete c;
    return nullptr;
}

}  // namespace

extern "C" {

moearc_ctx *moearc_ctx_create(void) {
    auto *c = new moearc_ctx();
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0 || hipGetDevice(&c->device) != hipSuccess)
        return release(c);
    // Default priority, in-order (the reference's in-order queue, kernels.cpp:806-810).
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) return release(c);
    const char *co_env = std::getenv("MOEARC_CODE_OBJECT");
    const std::string co = co_env ? std::string(co_env) : library_dir() + "/moearc_attn_gfx950.co";
    if (hipModuleLoad(&c->module, co.c_str()) != hipSuccess) {
        std::fprintf(stderr, "moearc: cannot load code object %s\n", co.c_str());
        return release(c);
    }
    const uint32_t zero = 0;
    if (hipMalloc((void **) &c->err_word, 256) != hipSuccess ||
        hipMemcpy(c->err_word, &zero, 4, hipMemcpyHostToDevice) != hipSuccess)
        return release(c);
    // The fixed record array's address in this module instance (per context, on its device). The
    // symbol's name on the host is not a device address; only this pointer is ever passed on.
    hipDeviceptr_t scratch = nullptr;
    size_t scratch_bytes = 0;
    if (hipModuleGetGlobal(&scratch, &scratch_bytes, c->module, "moearc_decode_scratch") != hipSuccess ||
        !scratch || scratch_bytes < (size_t) MOEARC_DECODE_SCRATCH_FLOATS * sizeof(float)) {
        std::fprintf(stderr, "moearc: code object %s lacks the decode record array\n", co.c_str());
        return release(c);
    }
    c->scratch = (float *) scratch;
    c->scratch_floats = scratch_bytes / sizeof(float);
    struct {
        hipFunction_t *slot;
        const char *name;
    } fns[] = {
        {&c->f_zero, "moearc_zero_k"},
        {&c->f_quant, "moearc_quantize_f16_k"},
        {&c->f_append, "moearc_kv_append_k"},
        {&c->f_append_chunk, "moearc_kv_append_chunk_k"},
        {&c->f_rope, "moearc_rope_k"},
        {&c->f_rope_f16, "moearc_rope_f16_k"},
        {&c->f_rope_append_chunk, "moearc_rope_kv_append_chunk_k"},
        {&c->f_rope_append64, "moearc_rope_kv_append_chunk64_k"},
        {&c->f_rope_qkv64, "moearc_rope_qkv_chunk64_k"},
        {&c->f_rope_sums64, "moearc_rope_qkv_sums64_k"},
        {&c->f_dec_general, "moearc_attn_decode_general_k"},
        {&c->f_dec_fast[0], "moearc_attn_decode_f16d64_k4w2t4"},
        {&c->f_dec_fast[1], "moearc_attn_decode_f16d64_k1w4t1"},
        {&c->f_dec_merge, "moearc_attn_decode_merge_p1"},
        {&c->f_add, "moearc_add_k"},
        {&c->f_read_floor, "moearc_read_floor_k"},
        {&c->f_mfma_floor, "moearc_mfma_floor_k"},
        {&c->f_mm[0][0], "moearc_matmul_q8_0_r1_k"},
        {&c->f_mm[0][1], "moearc_matmul_q8_0_r2_k"},
        {&c->f_mm[1][0], "moearc_matmul_f16_r1_k"},
        {&c->f_mm[1][1], "moearc_matmul_f16_r2_k"},
        {&c->f_mm[2][0], "moearc_matmul_q4_k_r1_k"},
        {&c->f_mm[2][1], "moearc_matmul_q4_k_r2_k"},
        {&c->f_mm[3][0], "moearc_matmul_q5_k_r1_k"},
        {&c->f_mm[3][1], "moearc_matmul_q5_k_r2_k"},
        {&c->f_mm[4][0], "moearc_matmul_mxfp4_r1_k"},
        {&c->f_mm[4][1], "moearc_matmul_mxfp4_r2_k"},
        {&c->f_mm[5][0], "moearc_matmul_q6_k_r1_k"},
        {&c->f_mm[5][1], "moearc_matmul_q6_k_r2_k"},
        {&c->f_mm2[0], "moearc_matmul2_q8_0_k"},
        {&c->f_mm2[1], "moearc_matmul2_f16_k"},
        {&c->f_mm2[2], "moearc_matmul2_q4_k_k"},
        {&c->f_mm2[3], "moearc_matmul2_q5_k_k"},
        {&c->f_mm2[4], "moearc_matmul2_q6_k_k"},
        {&c->f_mm2[5], "moearc_matmul2_mxfp4_k"},
        {&c->f_mm2w[0], "moearc_matmul2w_q8_0_k"},
        {&c->f_mm2w[1], "moearc_matmul2w_f16_k"},
        {&c->f_mm2w[2], "moearc_matmul2w_mxfp4_k"},
        {&c->f_bsums, "moearc_block_sums_k"},
        {&c->f_split, "moearc_split_f16_k"},
        {&c->f_split8, "moearc_split_f16_v8_k"},
        {&c->f_mm_reduce, "moearc_matmul_reduce_k"},
        {&c->f_mm_reduce4, "moearc_matmul_reduce4_k"},
    };
    for (auto &f : fns) {
        if (hipModuleGetFunction(f.slot, c->module, f.name) != hipSuccess) {
            std::fprintf(stderr, "moearc: code object %s lacks kernel %s\n", co.c_str(), f.name);
            return release(c);
        }
    }
    int merge_threads = 0;
    if (hipFuncGetAttribute(&merge_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->f_dec_merge) !=
            hipSuccess || merge_threads != MOEARC_MERGE_THREADS) {
        std::fprintf(stderr, "moearc: cannot read the merge kernel's work-group size\n");
        return release(c);
    }
    c->merge_threads = (unsigned) merge_threads;
    if (const char *pp = std::getenv("MOEARC_PREFILL_PRECISE")) c->prefill_precise = pp[0] == '1';
    if (const char *bf = std::getenv("MOEARC_BLOCK_FUSED")) c->block_fused = bf[0] != '0';
    for (int i = 0; i < 8; ++i) {
        const bool precise = i >= 4;
        char name[64];
        std::snprintf(name, sizeof(name), "moearc_attn_prefill_%sg%d", precise ? "precise_" : "", 1 << (i & 3));
        hipFunction_t *slot = precise ? &c->f_prefill_precise[i & 3] : &c->f_prefill[i & 3];
        if (hipModuleGetFunction(slot, c->module, name) != hipSuccess) {
            std::fprintf(stderr, "moearc: code object %s lacks kernel %s\n", co.c_str(), name);
            return release(c);
        }
    }
    for (int t = 0; t < 7; ++t) {
        for (int i = 0; i < 4; ++i) {
            if ((1u << i) > moearc_mv_ppl_max(kMvTypes[t])) continue;
            char name[64];
            std::snprintf(name, sizeof(name), "moearc_matvec_%s_p%u", kMvNames[t], 1u << i);
            if (hipModuleGetFunction(&c->f_mv[t][i], c->module, name) != hipSuccess) {
                std::fprintf(stderr, "moearc: code object %s lacks kernel %s\n", co.c_str(), name);
                return release(c);
            }
        }
    }
    if (const char *r = std::getenv("MOEARC_MATVEC_RPW")) c->mv_rpw_override = std::strtoul(r, nullptr, 10);
    if (const char *w = std::getenv("MOEARC_MATVEC_WAVES")) {
        const unsigned long v = std::strtoul(w, nullptr, 10);
        if (v == 4 || v == 8) c->mv_waves_override = (unsigned) v;
    }
    const char *ev = std::getenv("MOEARC_PROFILE_EVENTS");
    const char *ek = std::getenv("MOEARC_PROFILE_KERNELS");
    c->profile_kernels = ek && ek[0] == '1';
    c->profiling = (ev && ev[0] == '1') || c->profile_kernels;
    if (const char *w = std::getenv("MOEARC_DECODE_VARIANT")) {
        for (int i = 0; i < kNumDecodeVariants; ++i)
            if (std::strcmp(w, kDecodeVariants[i].name) == 0) c->decode_variant_override = i;
    }
    if (const char *s = std::getenv("MOEARC_DECODE_SPLIT")) c->split_override = std::strtoul(s, nullptr, 10);
    if (const char *pb = std::getenv("MOEARC_PF_BOOST")) {
        float x = 0.f, y = 0.f;
        if (std::sscanf(pb, "%f,%f", &x, &y) == 2) {
            c->pf_boost_a = x;
            c->pf_boost_b = y;
        }
    }
    {
        int ncu = 0;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, c->device) == hipSuccess && ncu > 0)
            c->n_cu = (unsigned) ncu;
    }
    if (const char *s = std::getenv("MOEARC_MM_WIDE")) c->mm_wide = std::strtoul(s, nullptr, 10) ? 1 : 0;
    if (const char *s = std::getenv("MOEARC_MM_SPLIT_WG")) c->mm_split_wg = (int) std::min(8ul, std::strtoul(s, nullptr, 10));
    return c;
}

void moearc_ctx_destroy(moearc_ctx *c) {
    if (!c) return;
    release(c);
}

// The host computes theta_scale as the reference does before its launch (kernels.cpp:1406).
static RopeParams rope_params(unsigned long n_dims, float freq_base, float freq_scale,
                              float ext_factor, float attn_factor, float corr_lo, float corr_hi,
                              int neox) {
    RopeParams r{};
    r.n_dims = (uint32_t) n_dims;
    r.neox = neox ? 1u : 0u;
    r.theta_scale = std::pow(freq_base, -2.0f / (float) n_dims);
    r.freq_scale = freq_scale;
    r.ext_factor = ext_factor;
    r.attn_factor = attn_factor;
    r.corr_lo = corr_lo;
    r.corr_hi = corr_hi;
    return r;
}

}  // extern "C"

namespace {

// moearc_rope's checks and launch, into f32 (f_rope) or binary16 (f_rope_f16) rows.
int rope_launch(moearc_ctx *c, hipFunction_t f, void *dst, const float *src, const int *pos,
                unsigned long n_tokens, unsigned long n_heads, unsigned long head_dim,
                unsigned long n_dims, float freq_base, float freq_scale, float ext_factor,
                float attn_factor, float corr_lo, float corr_hi, int neox) {
    if (!c || !dst || !src || !pos) return ERR;
    if (n_dims == 0 || n_dims % 2 != 0 || n_dims > head_dim) return ERR_ARG;
    if (n_tokens == 0 || n_heads == 0) return OK;
    if (head_dim > 0xFFFFFFFFul || n_heads > 0xFFFFFFFFul) return ERR_ARG;
    // threads over (token, pair slot); grid y over groups of ROPE_HEADS heads
    const uint64_t threads = (uint64_t) n_tokens * ((head_dim + 1) / 2);
    const uint64_t groups = (n_heads + ROPE_HEADS - 1) / ROPE_HEADS;
    if (threads / 256 >= 0xFFFFFFFFull || groups > 65535) return ERR_ARG;
    struct {
        void *dst;
        const float *src;
        const int *pos;
        uint64_t n_tokens;
        uint32_t n_heads, head_dim;
        RopeParams r;
    } a{dst, src, pos, n_tokens, (uint32_t) n_heads, (uint32_t) head_dim,
        rope_params(n_dims, freq_base, freq_scale, ext_factor, attn_factor, corr_lo, corr_hi, neox)};
    return launch2d(c, f, (unsigned) ((threads + 255) / 256), (unsigned) groups, 256, a,
                    nullptr, n_heads, head_dim, 0, "rope");
}

}  // namespace

extern "C" {

int moearc_rope(moearc_ctx *c, float *dst, const float *src, const int *pos,
                unsigned long n_tokens, unsigned long n_heads, unsigned long head_dim,
                unsigned long n_dims, float freq_base, float freq_scale, float ext_factor,
                float attn_factor, float corr_lo, float corr_hi, int neox) {
    if (!c) return ERR;
    return rope_launch(c, c->f_rope, dst, src, pos, n_tokens, n_heads, head_dim, n_dims, freq_base, freq_scale,
                       ext_factor, attn_factor, corr_lo, corr_hi, neox);
}

int moearc_rope_kv_append_chunk(moearc_ctx *c, void *k_pages, void *v_pages, const float *k,
                                const float *v, const int *pos, const unsigned int *page_ids,
                                const unsigned int *slots, unsigned long n_tok,
                                unsigned long n_kv_heads, unsigned long head_dim,
                                unsigned long page_tokens, unsigned long n_dims, float freq_base,
                                float freq_scale, float ext_factor, float attn_factor,
                                float corr_lo, float corr_hi, int neox, unsigned int kv_type) {
    if (!c || !k_pages || !v_pages || !k || !v || !pos || !page_ids || !slots) return ERR;
    if (n_dims == 0 || n_dims % 2 != 0 || n_dims > head_dim) return ERR_ARG;
    if (kv_type != 0u && kv_type != 1u) return ERR_ARG;
    if (page_tokens == 0 || n_kv_heads == 0 || head_dim == 0) return ERR_ARG;
    if (n_tok == 0) return OK;
    if (head_dim > 0xFFFFFFFFul || n_kv_heads > 0xFFFFFFFFul) return ERR_ARG;
    const RopeParams rp = rope_params(n_dims, freq_base, freq_scale, ext_factor, attn_factor, corr_lo, corr_hi, neox);
    // NeoX over all 64 channels into f16 pools, KV heads dividing 16, rows 16-byte aligned: whole
    // rows per lane group (moearc_rope_kv_append_chunk64_k)
    if (kv_type == 1u && neox && head_dim == 64 && n_dims == 64 && 16 % n_kv_heads == 0 &&
        ((uintptr_t) k | (uintptr_t) v) % 16 == 0 && ((uintptr_t) k_pages | (uintptr_t) v_pages) % 8 == 0) {
        const uint64_t wgs = (n_tok * n_kv_heads + 15) / 16;
        if (wgs >= 0xFFFFFFFFull) return ERR_ARG;
        struct {
            void *kp, *vp;
            const float *k, *v;
            const int *pos;
            const uint32_t *pages, *slots;
            uint64_t n_tok;
            uint32_t n_kv_heads;
            uint64_t pt;
            RopeParams r;
            uint32_t *err;
        } a{k_pages, v_pages, k, v, pos, page_ids, slots, n_tok, (uint32_t) n_kv_heads, page_tokens, rp, c->err_word};
        c->err_armed = true;
        return launch2d(c, c->f_rope_append64, (unsigned) wgs, 1, 256, a, "rope_kv_append_chunk", n_kv_heads, head_dim);
    }
    const uint64_t threads = (uint64_t) n_tok * ((head_dim + 1) / 2);
    const uint64_t groups = (n_kv_heads + ROPE_HEADS - 1) / ROPE_HEADS;
    if (threads / 256 >= 0xFFFFFFFFull || groups > 65535) return ERR_ARG;
    struct {
        void *kp, *vp;
        const float *k, *v;
        const int *pos;
        const uint32_t *pages, *slots;
        uint64_t n_tok;
        uint32_t n_kv_heads, head_dim;
        uint64_t pt;
        uint32_t kv_type;
        RopeParams r;
        uint32_t *err;
    } a{k_pages, v_pages, k, v, pos, page_ids, slots, n_tok, (uint32_t) n_kv_heads,
        (uint32_t) head_dim, page_tokens, kv_type, rp, c->err_word};
    c->err_armed = true;
    return launch2d(c, c->f_rope_append_chunk, (unsigned) ((threads + 255) / 256), (unsigned) groups,
                    256, a, "rope_kv_append_chunk", n_kv_heads, head_dim);
}

void *moearc_ctx_stream(moearc_ctx *c) { return c ? (void *) c->stream : nullptr; }

int moearc_profile_events_enabled(moearc_ctx *c) { return (c && c->profiling) ? 1 : 0; }

int moearc_profile_events_reset(moearc_ctx *c) {
    if (!c) return ERR;
    flush_events(c);
    c->totals.clear();
    return OK;
}

int moearc_profile_events_report(moearc_ctx *c, char *out, unsigned long cap) {
    if (!c || !out || cap == 0) return ERR;
    if (!c->profiling) {
        out[0] = '\0';
        return OK;
    }
    flush_events(c);
    unsigned long used = 0;
    for (const auto &t : c->totals) {
        char line[160];
        const int n = std::snprintf(line, sizeof(line), "%s %llu %llu\n", t.key.c_str(), t.ns, t.calls);
        if (n <= 0 || used + (unsigned long) n + 1 > cap) break;
        std::memcpy(out + used, line, (size_t) n);
        used += (unsigned long) n;
    }
    out[used] = '\0';
    return OK;
}

int moearc_sync(moearc_ctx *c) {
    if (!c) return ERR;
    if (hipStreamSynchronize(c->stream) != hipSuccess) return ERR;
    bool failed = c->deferred_error;
    c->deferred_error = false;
    if (c->err_armed) {
        c->err_armed = false;
        uint32_t word = 0;
        if (hipMemcpyAsync(&word, c->err_word, 4, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
            hipStreamSynchronize(c->stream) != hipSuccess)
            return ERR;
        if (word != 0) {
            const uint32_t zero = 0;
            if (hipMemcpyAsync(c->err_word, &zero, 4, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
                hipStreamSynchronize(c->stream) != hipSuccess)
                return ERR;
            failed = true;
        }
    }
    return failed ? ERR : OK;
}

int moearc_zero(moearc_ctx *c, float *dst, unsigned long n) {
    if (!c || !dst) return ERR;
    if (n == 0) return OK;
    const unsigned grid = (unsigned) std::min<unsigned long>((n + 255) / 256, 65536ul);
    struct {
        float *d;
        uint64_t n;
    } a{dst, n};
    return launch(c, c->f_zero, grid, 256, a, nullptr, n, 0, "zero");
}

int moearc_device_name(moearc_ctx *c, char *out, unsigned long cap) {
    if (!c || !out || cap == 0) return ERR;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, c->device) != hipSuccess) return ERR;
    char name[256] = {0};
    if (p.name[0]) std::snprintf(name, sizeof(name), "%s", p.name);
    else if (hipDeviceGetName(name, (int) sizeof(name), c->device) != hipSuccess || !name[0])
        std::snprintf(name, sizeof(name), "device %d", c->device);
    std::snprintf(out, cap, "%s (%s, %d CUs)", name, p.gcnArchName, p.multiProcessorCount);
    return OK;
}

void *moearc_alloc_device(moearc_ctx *c, unsigned long bytes) {
    if (!c) return nullptr;
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) return nullptr;
    return p;
}

void moearc_free_device(moearc_ctx *c, void *p) {
    if (!c || !p) return;
    // no return code in the reference's signature (ffi.rs:33): a failure surfaces at moearc_sync
    if (hipStreamSynchronize(c->stream) != hipSuccess || hipFree(p) != hipSuccess) c->deferred_error = true;
}

int moearc_copy_h2d(moearc_ctx *c, void *dst, const void *src, unsigned long bytes) {
    if (!c) return ERR;
    if (bytes == 0) return OK;
    if (!dst || !src) return ERR;
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream) != hipSuccess) return ERR;
    return hipStreamSynchronize(c->stream) == hipSuccess ? OK : ERR;
}

int moearc_copy_h2d_async(moearc_ctx *c, void *dst, const void *src, unsigned long bytes) {
    if (!c) return ERR;
    if (bytes == 0) return OK;
    if (!dst || !src) return ERR;
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream) == hipSuccess ? OK : ERR;
}

int moearc_copy_d2h(moearc_ctx *c, void *dst, const void *src, unsigned long bytes) {
    if (!c) return ERR;
    if (bytes == 0) return OK;
    if (!dst || !src) return ERR;
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream) != hipSuccess) return ERR;
    return hipStreamSynchronize(c->stream) == hipSuccess ? OK : ERR;
}

namespace {

// One matrix of a matvec launch: out[r] = W[r] . x (+ bias[r]) for r < rows.
struct MvJob {
    const void *w;
    const float *x;
    const float *bias;
    float *out;
    unsigned long rows;
    bool residual = false;  // out[r] += the result (out holds the residual)
};

constexpr unsigned kMvLdsCap = 64u * 1024u;  // dynamic LDS per work-group the launches stay under
// Rows per wave: enough that the launch is about one work-group per CU (256 on MI355X). Fewer,
// longer-lived waves measured faster than more, shorter ones at the projection shapes: each
// work-group stages the activation once, and a wave keeps two rows in flight.
constexpr unsigned long kMvCUs = 256ul;

// Shape checks shared by the matvec entry points (kernels.cpp:1053-1057): the type must be known
// and a row a whole number of blocks.
int mv_check(unsigned ty, unsigned long n_rows, unsigned long n_cols) {
    if (mv_type_index(ty) < 0) return ERR_ARG;
    if (n_cols % moearc_mv_be(ty) != 0) return ERR_ARG;
    if (n_rows > 0xFFFFFFFFul || n_cols >= 0x80000000ul) return ERR_ARG;
    return OK;
}

// Enqueue jobs[0..n) (all of weight type ty, n_cols columns) as one launch; n <= MOEARC_MV_MAX_SEG.
int mv_launch(moearc_ctx *c, unsigned ty, const MvJob *jobs, unsigned n, unsigned long n_cols,
              const char *what, unsigned long key_r, unsigned long key_m) {
    const int t = mv_type_index(ty);
    if (t < 0 || n == 0 || n > MOEARC_MV_MAX_SEG) return ERR_ARG;
    const uint32_t pe = moearc_mv_pe(ty);
    if (n_cols == 0) {  // empty rows: the sum is 0 (then the bias)
        for (unsigned i = 0; i < n; ++i) {
            if (!jobs[i].rows) continue;
            if (jobs[i].residual) {  // out += 0 (+ bias)
                if (jobs[i].bias)
                    if (const int rc = moearc_add(c, jobs[i].out, jobs[i].out, jobs[i].bias, jobs[i].rows)) return rc;
                continue;
            }
            const int rc = jobs[i].bias
                               ? (hipMemcpyAsync(jobs[i].out, jobs[i].bias, jobs[i].rows * 4ul,
                                                 hipMemcpyDeviceToDevice, c->stream) == hipSuccess ? OK : ERR)
                               : moearc_zero(c, jobs[i].out, jobs[i].rows);
            if (rc) return rc;
        }
        return OK;
    }
    const uint64_t pieces = (n_cols + pe - 1) / pe;
    uint32_t li = 0;  // pieces per lane 1 << li
    while ((64ull << li) < pieces && (2u << li) <= moearc_mv_ppl_max(ty)) ++li;
    const uint32_t ppl = 1u << li;
    const uint64_t slabs = (pieces + 64ull * ppl - 1) / (64ull * ppl);
    const uint64_t row_bytes = (uint64_t) n_cols / moearc_mv_be(ty) * moearc_mv_bb(ty);
    const uint64_t slab_bytes =
        slabs == 1 ? row_bytes : 64ull * ppl * pe * moearc_mv_bb(ty) / moearc_mv_be(ty);
    const unsigned wave_buf = moearc_mv_wave_buf(slab_bytes);
    const uint64_t x_lds = (pieces * (pe + 4u) * 4u + 15u) & ~15ull;
    unsigned waves = MOEARC_MV_MAX_WAVES, x_in_lds = 1;
    if (x_lds + (uint64_t) waves * wave_buf > kMvLdsCap) {
        if (x_lds + 4ull * wave_buf <= kMvLdsCap) {
            waves = 4;
        } else {
            x_in_lds = 0;
            if ((uint64_t) waves * wave_buf > kMvLdsCap) waves = 4;
        }
    }
    const uint64_t x_bytes = x_in_lds ? x_lds : 0;
    unsigned long total = 0;
    for (unsigned i = 0; i < n; ++i) total += jobs[i].rows;
    if (total == 0) return OK;
    if (c->mv_waves_override && x_lds * (x_in_lds ? 1 : 0) + (uint64_t) c->mv_waves_override * wave_buf <= kMvLdsCap)
        waves = c->mv_waves_override;
    const uint32_t rpw = (uint32_t) std::min<unsigned long>(
        64, c->mv_rpw_override ? c->mv_rpw_override
                               : std::max<unsigned long>(1, (total + kMvCUs * waves - 1) / (kMvCUs * waves)));
    MatvecArgs a{};
    uint64_t wgs = 0;
    for (unsigned i = 0; i < n; ++i) {
        a.w[i] = static_cast<const uint8_t *>(jobs[i].w);
        a.x[i] = jobs[i].x;
        a.bias[i] = jobs[i].bias ? jobs[i].bias : jobs[i].out;
        a.bias_mask |= jobs[i].bias ? 1u << i : 0u;
        a.res_mask |= jobs[i].residual ? 1u << i : 0u;
        a.out[i] = jobs[i].out;
        a.rows[i] = (uint32_t) jobs[i].rows;
        wgs += (jobs[i].rows + (uint64_t) waves * rpw - 1) / ((uint64_t) waves * rpw);
        if (wgs >= 0x7FFFFFFFull) return ERR_ARG;
        a.wg_end[i] = (uint32_t) wgs;
    }
    a.row_bytes = row_bytes;
    a.wave_buf = wave_buf;
    a.n_seg = n;
    a.n_cols = (uint32_t) n_cols;
    a.n_pieces = (uint32_t) pieces;
    a.n_slabs = (uint32_t) slabs;
    a.rpw = rpw;
    a.x_in_lds = x_in_lds;
    a.x_lds_bytes = (uint32_t) x_bytes;
    // Keys of the reference's matvec entry points (kernels.cpp:1057-1111, :1168-1196): "mvq <type>"
    // and "mvq_batched <type>" for the block formats, "mv_generic ... m1" for F32/F16 weights;
    // moearc_matvec_f32 is not tracked there (what == nullptr); this build's fused entry points
    // keep their own names with the type appended.
    char key[48], kname[48];
    const bool generic = ty == 0u || ty == 1u;
    const bool ref_entry = what && (std::strcmp(what, "mvq") == 0 || std::strcmp(what, "mvq_batched") == 0);
    if (ref_entry && generic) {
        std::snprintf(key, sizeof(key), "mv_generic");
        key_m = 1;
    } else if (what) {
        std::snprintf(key, sizeof(key), "%s %s", what, kMvKeys[t]);
    }
    std::snprintf(kname, sizeof(kname), "matvec %s", kMvKeys[t]);
    return launch2d(c, c->f_mv[t][li], (unsigned) wgs, 1, 64u * waves, a, what ? key : nullptr, key_r,
                    key_m, (unsigned) (x_bytes + (uint64_t) waves * wave_buf), kname);
}

}  // namespace

int moearc_matvec_q(moearc_ctx *c, unsigned int type_id, float *out, const void *w,
                    const float *x, unsigned long n_rows, unsigned long n_cols) {
    if (!c || !out || !w || !x) return ERR;
    if (const int rc = mv_check(type_id, n_rows, n_cols)) return rc;
    if (n_rows == 0) return OK;
    const MvJob j{w, x, nullptr, out, n_rows};
    return mv_launch(c, type_id, &j, 1, n_cols, "mvq", n_rows, 1);
}

int moearc_matvec_q_batched(moearc_ctx *c, unsigned int type_id, float *out, const void *const *w,
                            unsigned int n_mat, const float *x, unsigned long x_stride,
                            unsigned long n_rows, unsigned long n_cols) {
    if (!c || !out || !w || !x) return ERR;
    if (n_mat == 0 || n_rows == 0) return OK;
    if (n_mat > MOEARC_MV_MAX_SEG) return ERR_ARG;
    if (const int rc = mv_check(type_id, n_rows, n_cols)) return rc;
    MvJob jobs[MOEARC_MV_MAX_SEG];
    for (unsigned m = 0; m < n_mat; ++m) {
        if (!w[m]) return ERR;
        jobs[m] = MvJob{w[m], x + m * x_stride, nullptr, out + m * n_rows, n_rows};
    }
    return mv_launch(c, type_id, jobs, n_mat, n_cols, "mvq_batched", n_rows, n_mat);
}

int moearc_matvec_f32(moearc_ctx *c, float *out, const float *w, const float *x,
                      unsigned long n_rows, unsigned long n_cols) {
    if (!c || !out || !w || !x) return ERR;
    if (n_rows == 0) return OK;
    if (const int rc = mv_check(0, n_rows, n_cols)) return rc;
    const MvJob j{w, x, nullptr, out, n_rows};
    return mv_launch(c, 0, &j, 1, n_cols, nullptr, n_rows, 1);
}

int moearc_add(moearc_ctx *c, float *out, const float *a, const float *b, unsigned long n) {
    if (!c || !out || !a || !b) return ERR;
    if (n == 0) return OK;
    const unsigned grid = (unsigned) std::min<unsigned long>((n + 255) / 256, 65536ul);
    struct {
        float *o;
        const float *a, *b;
        uint64_t n;
    } args{out, a, b, n};
    return launch(c, c->f_add, grid, 256, args, nullptr, n, 0, "add");
}

int moearc_read_floor(moearc_ctx *c, unsigned int *out, const void *src, unsigned long bytes) {
    if (!c || !out || !src) return ERR;
    if (bytes == 0 || bytes % 16 != 0 || (uintptr_t) src % 16 != 0) return ERR_ARG;
    const uint64_t wgs = (bytes + 65535) / 65536;  // 64 KiB per work-group
    if (wgs > 0x7FFFFFFFull) return ERR_ARG;
    struct {
        unsigned int *o;
        const void *s;
        uint64_t n16;
    } args{out, src, bytes / 16};
    return launch(c, c->f_read_floor, (unsigned) wgs, 256, args, nullptr, bytes, 0, "read_floor");
}

int moearc_mfma_floor(moearc_ctx *c, float *out, const void *src, unsigned long n_wgs,
                      unsigned long iters) {
    if (!c || !out || !src) return ERR;
    if (n_wgs == 0 || n_wgs > 0x7FFFFFFFul / 4 || iters == 0 || iters % 4 != 0 || iters > 0x40000000ul ||
        (uintptr_t) src % 16 != 0)
        return ERR_ARG;
    struct {
        float *o;
        const void *s;
        uint32_t it;
    } args{out, src, (uint32_t) iters};
    return launch(c, c->f_mfma_floor, (unsigned) n_wgs, 256, args, nullptr, n_wgs, iters, "mfma_floor");
}

int moearc_attn_out(moearc_ctx *c, unsigned int type_id, float *h, const void *w, const float *bias,
                    const float *attn, unsigned long n_rows, unsigned long n_cols) {
    if (!c || !h || !w || !attn) return ERR;
    if (const int rc = mv_check(type_id, n_rows, n_cols)) return rc;
    if (n_rows == 0) return OK;
    MvJob j{w, attn, bias, h, n_rows, true};
    return mv_launch(c, type_id, &j, 1, n_cols, "attn_out", n_rows, 1);
}

int moearc_attn_qkv(moearc_ctx *c, const unsigned int *type_ids, float *const *out,
                    const void *const *w, const float *const *bias, const unsigned long *rows,
                    const float *x, unsigned long n_cols) {
    if (!c || !type_ids || !out || !w || !bias || !rows || !x) return ERR;
    for (int i = 0; i < 3; ++i) {
        if (rows[i] && (!out[i] || !w[i])) return ERR;
        if (const int rc = mv_check(type_ids[i], rows[i], n_cols)) return rc;
    }
    bool done[3] = {false, false, false};
    for (int i = 0; i < 3; ++i) {  // one launch per distinct weight type, in q, k, v order
        if (done[i]) continue;
        MvJob jobs[3];
        unsigned n = 0;
        for (int k = i; k < 3; ++k) {
            if (done[k] || type_ids[k] != type_ids[i]) continue;
            done[k] = true;
            if (rows[k]) jobs[n++] = MvJob{w[k], x, bias[k], out[k], rows[k]};
        }
        if (n == 0) continue;
        if (const int rc = mv_launch(c, type_ids[i], jobs, n, n_cols, "attn_qkv", n, 3)) return rc;
    }
    return OK;
}

int moearc_quantize_f16(moearc_ctx *c, void *dst, const float *src, unsigned long n) {
    if (!c || !dst || !src) return ERR;
    if (n == 0) return OK;
    const unsigned grid = (unsigned) std::min<unsigned long>((n + 255) / 256, 65536ul);
    struct {
        void *d;
        const float *s;
        uint64_t n;
    } a{dst, src, n};
    return launch(c, c->f_quant, grid, 256, a, nullptr, n, 0, "quantize_f16");
}

int moearc_kv_append(moearc_ctx *c, void *k_pages, void *v_pages, const float *k, const float *v,
                     unsigned int page_id, unsigned int slot, unsigned long n_kv_heads,
                     unsigned long head_dim, unsigned long page_tokens, unsigned int kv_type) {
    if (!c || !k_pages || !v_pages || !k || !v) return ERR;
    if (kv_type != 0u && kv_type != 1u) return ERR_ARG;
    if (page_tokens == 0 || slot >= page_tokens) return ERR_ARG;
    if (n_kv_heads == 0 || head_dim == 0) return ERR_ARG;
    const uint64_t row = (uint64_t) n_kv_heads * head_dim;
    struct {
        void *kp, *vp;
        const float *k, *v;
        uint64_t base, row;
        uint32_t kv_type;
    } a{k_pages, v_pages, k, v, ((uint64_t) page_id * page_tokens + slot) * row, row, kv_type};
    return launch(c, c->f_append, (unsigned) ((row + 255) / 256), 256, a, nullptr, n_kv_heads,
                  head_dim);
}

int moearc_kv_append_chunk(moearc_ctx *c, void *k_pages, void *v_pages, const float *k,
                           const float *v, const unsigned int *page_ids, const unsigned int *slots,
                           unsigned long n_tok, unsigned long n_kv_heads, unsigned long head_dim,
                           unsigned long page_tokens, unsigned int kv_type) {
    if (!c || !k_pages || !v_pages || !k || !v || !page_ids || !slots) return ERR;
    if (kv_type != 0u && kv_type != 1u) return ERR_ARG;
    if (page_tokens == 0 || n_kv_heads == 0 || head_dim == 0) return ERR_ARG;
    if (n_tok == 0) return OK;
    const uint64_t row = (uint64_t) n_kv_heads * head_dim;
    const uint64_t total = row * n_tok;
    if (total / 256 >= 0xFFFFFFFFull) return ERR_ARG;
    struct {
        void *kp, *vp;
        const float *k, *v;
        const uint32_t *pages, *slots;
        uint64_t n_tok, row, pt;
        uint32_t kv_type;
        uint32_t *err;
    } a{k_pages, v_pages, k, v, page_ids, slots, n_tok, row, page_tokens, kv_type, c->err_word};
    c->err_armed = true;
    return launch(c, c->f_append_chunk, (unsigned) ((total + 255) / 256), 256, a, "kv_append_chunk",
                  n_kv_heads, head_dim);
}

int moearc_attn_decode(moearc_ctx *c, float *out, const float *q, const void *k_pages,
                       const void *v_pages, const unsigned int *block_table, const float *sinks,
                       unsigned long n_heads, unsigned long n_kv_heads, unsigned long head_dim,
                       unsigned long kv_begin, unsigned long n_kv, unsigned long page_tokens,
                       float scale, unsigned int kv_type) {
    // Validation order of kernels.cpp:1842-1852.
    if (!c || !out || !q || !k_pages || !v_pages || !block_table) return ERR;
    if (kv_type != 0u && kv_type != 1u) return ERR_ARG;
    if (n_heads == 0 || n_kv_heads == 0 || head_dim == 0 || n_kv == 0 || page_tokens == 0)
        return ERR_ARG;
    if (n_heads % n_kv_heads != 0) return ERR_ARG;
    if (kv_begin >= n_kv) return ERR_ARG;
    if (head_dim > 1024) return ERR_ARG;
    if (n_kv > 0xFFFFFFFFul) return ERR_ARG;  // keys are indexed in 32 bits on the device
    SpanList spans;
    spans.begin0 = (uint32_t) kv_begin;
    spans.end0 = (uint32_t) n_kv;
    spans.n = 1;
    const unsigned long bt_stride = (n_kv + page_tokens - 1) / page_tokens;
    return decode_launch(c, out, 0u, q, k_pages, v_pages, block_table, bt_stride, spans, sinks,
                         n_heads, n_kv_heads, head_dim, page_tokens, scale, kv_type);
}

int moearc_attn_decode_batched(moearc_ctx *c, void *out, unsigned int out_type, const float *q,
                               const void *k_pages, const void *v_pages,
                               const unsigned int *block_tables, unsigned long bt_stride,
                               const unsigned int *kv_begin, const unsigned int *n_kv,
                               const float *sinks, unsigned long n_seqs, unsigned long n_heads,
                               unsigned long n_kv_heads, unsigned long head_dim,
                               unsigned long page_tokens, float scale, unsigned int kv_type) {
    if (!c || !out || !q || !k_pages || !v_pages || !block_tables || !kv_begin || !n_kv) return ERR;
    if (kv_type != 0u && kv_type != 1u) return ERR_ARG;
    if (out_type != MOEARC_OUT_F32 && out_type != MOEARC_OUT_F16) return ERR_ARG;
    if (n_seqs == 0 || n_heads == 0 || n_kv_heads == 0 || head_dim == 0 || page_tokens == 0)
        return ERR_ARG;
    if (n_heads % n_kv_heads != 0) return ERR_ARG;
    if (head_dim > 1024) return ERR_ARG;
    for (unsigned long b = 0; b < n_seqs; ++b) {
        if (n_kv[b] == 0 || kv_begin[b] >= n_kv[b]) return ERR_ARG;
        if ((n_kv[b] + page_tokens - 1) / page_tokens > bt_stride) return ERR_ARG;
    }
    SpanList spans;
    spans.kv_begin = kv_begin;
    spans.n_kv = n_kv;
    spans.n = n_seqs;
    return decode_launch(c, out, out_type, q, k_pages, v_pages, block_tables, bt_stride, spans,
                         sinks, n_heads, n_kv_heads, head_dim, page_tokens, scale, kv_type);
}

int moearc_attn_decode_batched_noalloc(moearc_ctx *c, void *out, unsigned int out_type, const float *q,
                                       const void *k_pages, const void *v_pages,
                                       const unsigned int *block_tables, unsigned long bt_stride,
                                       const unsigned int *kv_begin, const unsigned int *n_kv,
                                       const float *sinks, unsigned long n_seqs, unsigned long n_heads,
                                       unsigned long n_kv_heads, unsigned long head_dim,
                                       unsigned long page_tokens, float scale, unsigned int kv_type) {
    // The checks and kernels of moearc_attn_decode_batched; the split records go to the code
    // object's fixed array (no hipMalloc, hipFree, event or host allocation), which a call must fit.
    if (!c || !out || !q || !k_pages || !v_pages || !block_tables || !kv_begin || !n_kv) return ERR;
    if (kv_type != 0u && kv_type != 1u) return ERR_ARG;
    if (out_type != MOEARC_OUT_F32 && out_type != MOEARC_OUT_F16) return ERR_ARG;
    if (n_seqs == 0 || n_heads == 0 || n_kv_heads == 0 || head_dim == 0 || page_tokens == 0)
        return ERR_ARG;
    if (n_heads % n_kv_heads != 0) return ERR_ARG;
    if (head_dim > 1024) return ERR_ARG;
    for (unsigned long b = 0; b < n_seqs; ++b) {
        if (n_kv[b] == 0 || kv_begin[b] >= n_kv[b]) return ERR_ARG;
        if ((n_kv[b] + page_tokens - 1) / page_tokens > bt_stride) return ERR_ARG;
    }
    if (!c->scratch) return ERR;
    SpanList spans;
    spans.kv_begin = kv_begin;
    spans.n_kv = n_kv;
    spans.n = n_seqs;
    RecordSpace rs;
    rs.fixed = c->scratch;
    rs.cap = c->scratch_floats;
    ++c->quiet;
    const int rc = decode_launch(c, out, out_type, q, k_pages, v_pages, block_tables, bt_stride, spans,
                                 sinks, n_heads, n_kv_heads, head_dim, page_tokens, scale, kv_type, rs);
    --c->quiet;
    return rc;
}

}  // extern "C"

namespace {

// The single-f16 kernels multiply each f32 score by scale*log2(e) after masking keys with -inf,
// which needs a positive finite scale; any other scale takes the precise kernels.
bool prefill_is_fast(const moearc_ctx *c, float scale) {
    const float c2 = scale * 1.4426950408889634f;
    return !c->prefill_precise && c2 > 0.0f && c2 <= 3.0e38f;
}

// moearc_attn_prefill's checks and launch; out_lo (f16 output, default kernels only) also takes
// the low halves of the chunk product's activation split.
int prefill_launch(moearc_ctx *c, void *out, unsigned int out_type, uint16_t *out_lo, const void *q,
                   const void *k_pages, const void *v_pages, const unsigned int *block_table,
                   const float *sinks, unsigned long n_q, unsigned long pos0,
                   unsigned long n_swa, unsigned long n_heads, unsigned long n_kv_heads,
                   unsigned long head_dim, unsigned long page_tokens, float scale,
                   unsigned int kv_type) {
    if (!c || !out || !q || !k_pages || !v_pages || !block_table) return ERR;
    if (kv_type != 1u) return ERR_ARG;
    if (out_type != MOEARC_OUT_F32 && out_type != MOEARC_OUT_F16) return ERR_ARG;
    if (n_q == 0 || n_heads == 0 || n_kv_heads == 0 || head_dim != 64 || !is_pow2(page_tokens))
        return ERR_ARG;
    if (n_heads % n_kv_heads != 0) return ERR_ARG;
    const unsigned long group = n_heads / n_kv_heads;
    if (group != 1 && group != 2 && group != 4 && group != 8) return ERR_ARG;
    if (pos0 + n_q > 0xFFFFFFFFul) return ERR_ARG;
    const int gi = group == 1 ? 0 : group == 2 ? 1 : group == 4 ? 2 : 3;
    const float scale_log2e = scale * 1.4426950408889634f;
    const bool precise = !prefill_is_fast(c, scale);
    if (out_lo && (precise || out_type != MOEARC_OUT_F16)) return ERR_ARG;
    hipFunction_t f = precise ? c->f_prefill_precise[gi] : c->f_prefill[gi];
    if (!f) return ERR;
    PrefillArgs a{};
    a.q = (const uint16_t *) q;
    a.k_pages = (const uint16_t *) k_pages;
    a.v_pages = (const uint16_t *) v_pages;
    a.block_table = block_table;
    a.sinks = sinks;
    a.out = out;
    a.n_q = (uint32_t) n_q;
    a.pos0 = (uint32_t) pos0;
    a.n_swa = (uint32_t) std::min<unsigned long>(n_swa, 0xFFFFFFFFul);
    a.n_heads = (uint32_t) n_heads;
    a.n_kv_heads = (uint32_t) n_kv_heads;
    a.group = (uint32_t) group;
    a.pt_shift = log2u(page_tokens);
    a.out_f16 = out_type;
    a.scale_log2e = scale_log2e;
    // query rows (token x head) per work-group
    const uint32_t rows_per_tile = precise ? MOEARC_PREFILL_ROWS : MOEARC_PREFILL_FAST_ROWS;
    const uint64_t rows = (uint64_t) n_q * group;
    a.n_qtiles = (uint32_t) ((rows + rows_per_tile - 1) / rows_per_tile);
    a.out_lo = out_lo;
    const uint64_t wgs = (uint64_t) a.n_qtiles * n_kv_heads;
    a.pair_half = c->n_cu && wgs == 2ull * c->n_cu ? c->n_cu : 0u;
    a.boost_a = c->pf_boost_a;
    a.boost_b = c->pf_boost_b;
    if (wgs > 0x7FFFFFFFull) return ERR_ARG;
    return launch(c, f, (unsigned) wgs, MOEARC_PREFILL_THREADS, a, "attn_prefill",
                  n_heads, head_dim);
}

}  // namespace

extern "C" {

int moearc_attn_prefill(moearc_ctx *c, void *out, unsigned int out_type, const void *q,
                        const void *k_pages, const void *v_pages, const unsigned int *block_table,
                        const float *sinks, unsigned long n_q, unsigned long pos0,
                        unsigned long n_swa, unsigned long n_heads, unsigned long n_kv_heads,
                        unsigned long head_dim, unsigned long page_tokens, float scale,
                        unsigned int kv_type) {
    return prefill_launch(c, out, out_type, nullptr, q, k_pages, v_pages, block_table, sinks, n_q, pos0, n_swa,
                          n_heads, n_kv_heads, head_dim, page_tokens, scale, kv_type);
}


}  // extern "C"

namespace {

constexpr uint64_t kMmCUs = 256;  // compute units the chunk product's launch shapes are sized for

// The reduction launch's arguments: the product's (y, bias, residual flag, slice sums) and the
// slice count.
struct MmReduceLaunch {
    MatmulArgs a;
    uint32_t n_slices;
    uint32_t pad;
};
// moearc_matmul_reduce_k(MatmulArgs a, uint32_t n_slices): the count follows the struct directly
static_assert(offsetof(MmReduceLaunch, n_slices) == sizeof(MatmulArgs), "reduce kernel argument layout");
static_assert(sizeof(MatmulArgs) % 8 == 0, "MatmulArgs is passed by value as 8-byte aligned kernel arguments");

// Chunk-product formats: index into f_mm, or -1.
int mm_index(unsigned ty) {
    return ty == 8u ? 0 : ty == 1u ? 1 : ty == 12u ? 2 : ty == 13u ? 3 : ty == 39u ? 4 : ty == 14u ? 5 : -1;
}

int mm_check(unsigned ty, const void *w, unsigned long n_tok, unsigned long n_rows, unsigned long n_cols) {
    if (mm_index(ty) < 0) return ERR_ARG;
    if (n_cols % 32 != 0 || n_cols % moearc_mv_be(ty) != 0 || ((uintptr_t) w & 1u) ||
        n_rows >= 0x80000000ul || n_tok >= 0x80000000ul || n_cols >= 0x80000000ul)
        return ERR_ARG;
    return OK;
}

// One matrix of a chunk-product launch: y (row stride y_stride) = W x (+ bias), W rows x n_cols.
struct MmMat {
    const void *w;
    const float *bias;
    float *y;
    unsigned long y_stride, rows;
};

// A split product's k-slice sums, left to a consumer that adds them itself (in slice order, then
// the bias, as moearc_matmul_reduce_k does): matrix i's slice z at part + z * stride + off[i],
// [t][r] with row stride `rows`. slices 0: the product was not split and wrote y itself.
struct MmSums {
    const float *part = nullptr;
    uint64_t stride = 0, off[MOEARC_MM_MAX_SEG] = {};
    uint32_t slices = 0;
};

// y = W x for n_mat matrices of one weight type over the same chunk x, given as its f16 split
// (xh, xl) of n_tok x n_cols, in one launch (plus the split-K reduction, unless `sums` takes the
// slices' sums instead; y is then not written).
int mm_launch(moearc_ctx *c, unsigned ty, const MmMat *m, unsigned n_mat, const uint16_t *xh, const uint16_t *xl,
              const float *xs, unsigned long n_tok, unsigned long n_cols, const char *what,
              bool accumulate = false, MmSums *sums = nullptr) {
    if (sums) *sums = MmSums{};
    if (n_mat == 0 || n_mat > MOEARC_MM_MAX_SEG) return ERR;
    MatmulArgs a{};
    a.accumulate = accumulate ? 1u : 0u;
    a.xh = xh;
    a.xl = xl;
    a.xs = xs;
    a.cols = (uint32_t) n_cols;
    a.n_tok = (uint32_t) n_tok;
    a.n_seg = n_mat;
    unsigned long n_rows = 0, tiles128 = 0, tiles256 = 0;
    for (unsigned i = 0; i < n_mat; ++i) {
        n_rows += m[i].rows;
        tiles128 += (m[i].rows + 127) / 128;
        tiles256 += (m[i].rows + 255) / 256;
    }
    // Every format over chunks of at least 64 tokens: 128 x 128 tiles on the 32x32x16 MFMA
    // (matmul2.hip; Q8_0 and MXFP4 weights arrive there in pairs of k-blocks, so their rows must
    // hold an even number of them). Otherwise 32 rows per wave halves the activation loads per MFMA, but only
    // pays while the launch still has about two work-groups per CU; shorter chunks take 16.
    hipFunction_t f;
    unsigned long rows_per_tile;
    unsigned gy;
    const bool pairs = ty == 8u || ty == 39u;
    const bool mm2 = (ty == 1u || ty == 12u || ty == 13u || ty == 14u || (pairs && (n_cols / 32) % 2 == 0)) &&
                     n_tok >= 64;
    // F16, Q8_0 and MXFP4 take work-groups of eight waves over 128 tokens x 256 rows (one per CU)
    // when those tiles alone cover every CU in whole rounds, the last at least three quarters
    // full: each k-block's copies into LDS then serve twice the rows, and the copies' volume is
    // what the CU pays for beside the MFMAs (at gpt-oss's attn_q over 2048 tokens, 256 tiles: F16
    // -20%, Q8_0 -4%, MXFP4 -6%). With fewer tiles than CUs, for the K-quants, and for a last
    // round mostly empty (the 2048-token block's q/k/v product, 320 tiles: +7% per block, its 64
    // last work-groups each alone on a CU for a whole wide tile) the 128 x 128 form is faster.
    const uint64_t wt = tiles256 * ((n_tok + 127) / 128);
    const bool wide = mm2 && (ty == 1u || ty == 8u || ty == 39u) &&
                      (c->mm_wide > 0 ||
                       (c->mm_wide < 0 && wt >= kMmCUs && (wt % kMmCUs == 0 || wt % kMmCUs >= kMmCUs * 3 / 4)));
    unsigned threads = 256;
    const int mm2_i = ty == 8u ? 0 : ty == 1u ? 1 : ty == 12u ? 2 : ty == 13u ? 3 : ty == 14u ? 4 : 5;
    if (wide) {
        f = c->f_mm2w[ty == 8u ? 0 : ty == 1u ? 1 : 2];
        rows_per_tile = 256;
        threads = 512;
        gy = (unsigned) ((n_tok + 127) / 128);
    } else if (mm2) {
        f = c->f_mm2[mm2_i];
        rows_per_tile = 128;
        gy = (unsigned) ((n_tok + 127) / 128);
    } else {
        const unsigned long tok_groups = (n_tok + MOEARC_MM_TOKENS - 1) / MOEARC_MM_TOKENS;
        const int r2 = tiles128 * tok_groups >= 512 ? 1 : 0;
        f = c->f_mm[mm_index(ty)][r2];
        rows_per_tile = r2 ? 128 : 64;
        gy = (unsigned) tok_groups;
    }
    uint64_t tile_end = 0, part_off = 0;
    for (unsigned i = 0; i < n_mat; ++i) {
        MatmulSeg &g = a.seg[i];
        g.w = static_cast<const uint8_t *>(m[i].w);
        g.bias = m[i].bias;
        g.y = m[i].y;
        g.row_bytes = (uint64_t) n_cols / moearc_mv_be(ty) * moearc_mv_bb(ty);
        g.rows = (uint32_t) m[i].rows;
        g.y_stride = (uint32_t) m[i].y_stride;
        g.part_off = part_off;
        tile_end += (m[i].rows + rows_per_tile - 1) / rows_per_tile;
        g.tile_end = (uint32_t) tile_end;
        part_off += (uint64_t) n_tok * m[i].rows;
    }
    a.part_stride = part_off;
    const unsigned gx = (unsigned) tile_end;
    // Split-K. A tile grid of at most one work-group per CU leaves most of the device idle while
    // each work-group walks the whole reduction (a 128-token chunk's k and v projections at gpt-oss
    // shapes are 4 work-groups), so the reduction is cut into slices of at least 4 k-blocks over a
    // third grid dimension, whose sums a second launch adds in slice order, with the bias and the
    // residual. The grid takes at most `aim` work-groups per CU: one for chunks of one or two
    // 128-token tiles and two above (measured on gpt-oss blocks: at 128 and 256 tokens the
    // reduction's traffic, which grows with the slices, outweighs a second work-group per CU; at 512
    // the reverse); MOEARC_MM_SPLIT_WG sets the aim. Rounding the slice count down keeps every CU's
    // share equal: rounded up, the grid's last work-groups double up on some CUs, which then set the
    // time (q/k/v at gpt-oss shapes, 5,120 rows: 256 tokens 41.7-42.2 -> 37.7-39.3 µs, 128 tokens
    // 27.0-27.7 -> 25.8-26.9). K-quant slices start on a 256-element super-block (a multiple of 8
    // k-blocks), matmul2.hip's Q8_0 and MXFP4 slices on a pair.
    const uint64_t nb = n_cols / 32, tiles = (uint64_t) gx * gy;
    const uint64_t gran = (ty == 12u || ty == 13u || ty == 14u) ? 8 : (mm2 && pairs) ? 2 : 1;
    uint64_t slices = 1, kb_per = nb;
    const uint64_t aim = c->mm_split_wg >= 0 ? (uint64_t) c->mm_split_wg : (gy <= 2 || wide) ? 1 : 2;
    if (tiles <= kMmCUs && nb >= 8 && aim) {
        const uint64_t want = std::max<uint64_t>(1, std::min<uint64_t>(aim * kMmCUs / tiles, nb / 4));
        kb_per = (nb + want - 1) / want;
        kb_per = (kb_per + gran - 1) / gran * gran;
        slices = (nb + kb_per - 1) / kb_per;
    }
    a.kb_per = (uint32_t) kb_per;
    if (slices < 2) return launch2d(c, f, gx, gy, threads, a, what, n_rows, n_tok);
    const size_t part = (size_t) slices * a.part_stride;
    if (part > c->mm_part_floats) {
        if (c->mm_part) {
            if (hipStreamSynchronize(c->stream) != hipSuccess || hipFree(c->mm_part) != hipSuccess) return ERR;
            c->mm_part = nullptr;
            c->mm_part_floats = 0;
        }
        if (hipMalloc((void **) &c->mm_part, part * sizeof(float)) != hipSuccess) return ERR;
        c->mm_part_floats = part;
    }
    a.part = c->mm_part;
    // one bracket for the call (the product and its reduction), as for a single launch
    hipEvent_t call0 = nullptr;
    if (what && tracks(c, what) && (call0 = take_event(c))) {
        if (hipEventRecord(call0, c->stream) != hipSuccess) {
            c->event_pool.push_back(call0);
            call0 = nullptr;
        }
    }
    ++c->scope_depth;
    int rc = launch3d(c, f, gx, gy, (unsigned) slices, threads, a, what, n_rows, n_tok);
    if (rc == OK && sums && !accumulate) {
        sums->part = a.part;
        sums->stride = a.part_stride;
        for (unsigned i = 0; i < n_mat; ++i) sums->off[i] = a.seg[i].part_off;
        sums->slices = (uint32_t) slices;
    } else if (rc == OK) {
        const uint64_t n = a.part_stride;
        bool by4 = n % 4 == 0 && (uintptr_t) a.part % 16 == 0;
        for (unsigned i = 0; i < n_mat; ++i)
            by4 = by4 && m[i].rows % 4 == 0 && m[i].y_stride % 4 == 0 && (uintptr_t) m[i].y % 16 == 0 &&
                  (uintptr_t) m[i].bias % 16 == 0;  // part_off: sums of n_tok * rows
        const uint64_t lanes = by4 ? n / 4 : n;
        rc = launch2d(c, by4 ? c->f_mm_reduce4 : c->f_mm_reduce, (unsigned) std::min<uint64_t>((lanes + 255) / 256, 65536),
                      1, 256, MmReduceLaunch{a, (uint32_t) slices, 0u}, nullptr, n_rows, n_tok, 0, "matmul_reduce");
    }
    --c->scope_depth;
    if (call0) record_bracket(c, call0, what, n_rows, n_tok);
    return rc;
}

// Whether a chunk product of this weight type reads the activation's block sums (the K-quants'
// mins: Q4_K, Q5_K).
bool mm_needs_sums(unsigned ty) { return ty == 12u || ty == 13u; }

// The f16 hi / lo split of x (n floats, n a multiple of 32) into the context's buffer, and its
// 32-element block sums when `sums` (else *xs points at space the products do not read).
// The split's buffers in the context's workspace (grown on demand): hi, lo, then n / 32 floats.
int mm_split_space(moearc_ctx *c, size_t n, uint16_t **xh, uint16_t **xl, float **xs) {
    const size_t halves = 2 * n + n / 16;  // hi, lo, then n / 32 floats
    if (halves > c->mm_ws_halves) {
        if (c->mm_ws) {
            if (hipStreamSynchronize(c->stream) != hipSuccess || hipFree(c->mm_ws) != hipSuccess) return ERR;
            c->mm_ws = nullptr;
            c->mm_ws_halves = 0;
        }
        if (hipMalloc((void **) &c->mm_ws, halves * sizeof(uint16_t)) != hipSuccess) return ERR;
        c->mm_ws_halves = halves;
    }
    *xh = c->mm_ws;
    *xl = c->mm_ws + n;
    *xs = (float *) (c->mm_ws + 2 * n);  // 4-byte aligned: n is a multiple of 32
    return OK;
}

int mm_split(moearc_ctx *c, const float *x, size_t n, uint16_t **xh, uint16_t **xl, float **xs, bool sums) {
    if (const int rc = mm_split_space(c, n, xh, xl, xs)) return rc;
    struct {
        const float *x;
        float *xs;
        uint64_t n;
    } bs{x, *xs, n / 32};
    if (sums)
        if (const int rc = launch(c, c->f_bsums, (unsigned) std::min<size_t>((n / 32 + 255) / 256, 65536), 256,
                                  bs, "block_sums", n / 32, 0))
            return rc;
    struct {
        const float *x;
        uint16_t *hi, *lo;
        uint64_t n;
    } a{x, *xh, *xl, n};
    // eight elements per thread when x allows 16-byte loads (hi and lo are: n is a multiple of 32)
    if ((uintptr_t) x % 16 == 0) {
        a.n = n / 8;
        return launch(c, c->f_split8, (unsigned) std::min<size_t>((n / 8 + 255) / 256, 65536), 256, a, "split_f16",
                      n, 0);
    }
    return launch(c, c->f_split, (unsigned) std::min<size_t>((n + 255) / 256, 65536), 256, a, "split_f16", n, 0);
}

}  // namespace

int moearc_matmul_q(moearc_ctx *c, unsigned int type_id, float *y, const void *w, const float *x,
                    const float *bias, unsigned long n_tok, unsigned long n_rows, unsigned long n_cols) {
    if (!c || !y || !w || !x) return ERR;
    if (const int rc = mm_check(type_id, w, n_tok, n_rows, n_cols)) return rc;
    if (n_rows == 0 || n_tok == 0) return OK;
    uint16_t *xh, *xl;
    float *xs;
    if (const int rc = mm_split(c, x, n_tok * n_cols, &xh, &xl, &xs, mm_needs_sums(type_id))) return rc;
    const MmMat mat{w, bias, y, n_rows, n_rows};
    return mm_launch(c, type_id, &mat, 1, xh, xl, xs, n_tok, n_cols, "matmul");
}

namespace {

// Run jobs[0..n) (one weight type) in launches of at most MOEARC_MV_MAX_SEG matrix-vector products.
int mv_launch_all(moearc_ctx *c, unsigned ty, const std::vector<MvJob> &jobs, unsigned long n_cols,
                  const char *what) {
    for (size_t i = 0; i < jobs.size(); i += MOEARC_MV_MAX_SEG) {
        const unsigned n = (unsigned) std::min<size_t>(MOEARC_MV_MAX_SEG, jobs.size() - i);
        if (const int rc = mv_launch(c, ty, jobs.data() + i, n, n_cols, what, jobs[i].rows, n)) return rc;
    }
    return OK;
}

}  // namespace

int moearc_attn_block_chunk(moearc_ctx *c, const moearc_attn_block *b, float *h, const float *x,
                            unsigned long n_tok, unsigned long pos0, const int *pos,
                            const unsigned int *page_ids, const unsigned int *slots) {
    if (!c || !b || !h || !x || !pos || !page_ids || !slots) return ERR;
    if (n_tok == 0) return OK;
    for (int i = 0; i < 4; ++i)
        if (!b->w[i]) return ERR;
    if (!b->k_pages || !b->v_pages || !b->block_table) return ERR;
    const unsigned long E = b->n_embd, H = b->n_head, G = b->n_head_kv, D = b->head_dim;
    if (H == 0 || G == 0 || D == 0 || E == 0 || H % G != 0) return ERR_ARG;
    const unsigned long q_rows = H * D, kv_rows = G * D;
    // the projections' shape checks, then the prefill's, before anything is enqueued
    for (int i = 0; i < 3; ++i)
        if (const int rc = mv_check(b->w_type[i], i == 0 ? q_rows : kv_rows, E)) return rc;
    if (const int rc = mv_check(b->w_type[3], E, q_rows)) return rc;
    const unsigned long group = H / G;
    if (D != 64 || !is_pow2(b->page_tokens) || (group != 1 && group != 2 && group != 4 && group != 8) ||
        pos0 + n_tok > 0xFFFFFFFFul || b->n_rot == 0 || b->n_rot % 2 != 0 || b->n_rot > D)
        return ERR_ARG;
    // A windowed block read through a ring: the chunk's K/V are written before its queries attend,
    // so while the first query attends the live keys run from its window start to the chunk's last
    // token, n_tok + n_swa - 1 of them; a smaller ring would let later tokens overwrite keys that
    // earlier rows still read.
    if (b->n_swa > 0 && b->ring_pages > 0 &&
        (unsigned long long) n_tok + b->n_swa - 1 > (unsigned long long) b->ring_pages * b->page_tokens)
        return ERR_ARG;

    // working memory: q, k, v, rotated q, f16 q, attention output, projection
    const size_t nq = n_tok * q_rows, nkv = n_tok * kv_rows;
    const size_t floats = nq + 2 * nkv + nq + (nq + 1) / 2 + nq + n_tok * E;
    if (floats * sizeof(float) > c->blk_ws_bytes) {
        if (c->blk_ws) {
            if (hipStreamSynchronize(c->stream) != hipSuccess || hipFree(c->blk_ws) != hipSuccess) return ERR;
            c->blk_ws = nullptr;
            c->blk_ws_bytes = 0;
        }
        if (hipMalloc((void **) &c->blk_ws, floats * sizeof(float)) != hipSuccess) return ERR;
        c->blk_ws_bytes = floats * sizeof(float);
    }
    float *q = c->blk_ws, *k = q + nq, *v = k + nkv, *qr = v + nkv;
    uint16_t *q16 = (uint16_t *) (qr + nq);
    float *att = qr + nq + (nq + 1) / 2, *proj = att + nq;

    // RoPE of q (written as f16 for the prefill kernel when there is a chunk: the values
    // moearc_quantize_f16 would make of the f32 rotation); RoPE of K fused with the K/V append.
    // With NeoX over all 64 channels and head counts that divide 16 or are multiples of it, both
    // go out as one launch (moearc_rope_qkv_chunk64_k), with the same results.
    const bool chunk = n_tok > 1;
    auto rows16 = [](unsigned long nh) { return nh != 0 && (16 % nh == 0 || nh % 16 == 0); };
    void *qdst = chunk ? (void *) q16 : (void *) qr;
    const bool rope_one = c->block_fused && D == 64 && b->n_rot == 64 && rows16(H) && rows16(G) &&
                          H <= 0xFFFFFFFFul &&
                          ((uintptr_t) q | (uintptr_t) qdst | (uintptr_t) k | (uintptr_t) v) % 16 == 0 &&
                          ((uintptr_t) b->k_pages | (uintptr_t) b->v_pages) % 8 == 0 &&
                          (n_tok * (H + G) + 15) / 16 < 0xFFFFFFFFull;
    // When that launch follows a split q/k/v product of one weight type, it adds the product's
    // k-slice sums and biases itself (moearc_rope_qkv_sums64_k) in place of the reduction launch:
    // one launch less, the same values.
    MmSums qkv_sums;

    // q, k, v (+ biases). A chunk of several tokens whose weights the MFMA product takes runs
    // as one matrix product per projection (the activation split once); the rest as every
    // (token, projection) pair through the batched matvec, grouped by weight type.
    const bool mm_qkv = n_tok >= 2 && E % 32 == 0 &&
                        mm_check(b->w_type[0], b->w[0], n_tok, q_rows, E) == OK &&
                        mm_check(b->w_type[1], b->w[1], n_tok, kv_rows, E) == OK &&
                        mm_check(b->w_type[2], b->w[2], n_tok, kv_rows, E) == OK;
    if (mm_qkv) {
        uint16_t *xh, *xl;
        float *xs;
        const bool sums = mm_needs_sums(b->w_type[0]) || mm_needs_sums(b->w_type[1]) || mm_needs_sums(b->w_type[2]);
        if (const int rc = mm_split(c, x, n_tok * E, &xh, &xl, &xs, sums)) return rc;
        float *outs[3] = {q, k, v};
        const unsigned long rows[3] = {q_rows, kv_rows, kv_rows};
        // the projections of one weight type in one launch (a block's q, k and v usually share it)
        bool done[3] = {false, false, false};
        for (int i = 0; i < 3; ++i) {
            if (done[i]) continue;
            MmMat mats[3];
            unsigned n = 0;
            for (int j = i; j < 3; ++j) {
                if (done[j] || b->w_type[j] != b->w_type[i]) continue;
                done[j] = true;
                mats[n++] = MmMat{b->w[j], b->bias[j], outs[j], rows[j], rows[j]};
            }
            if (const int rc = mm_launch(c, b->w_type[i], mats, n, xh, xl, xs, n_tok, E, "attn_qkv_mm", false,
                                         rope_one && n == 3 ? &qkv_sums : nullptr))
                return rc;
        }
    } else {
        float *outs[3] = {q, k, v};
        const unsigned long rows[3] = {q_rows, kv_rows, kv_rows};
        bool done[3] = {false, false, false};
        for (int i = 0; i < 3; ++i) {
            if (done[i]) continue;
            std::vector<MvJob> jobs;
            for (int j = i; j < 3; ++j) {
                if (done[j] || b->w_type[j] != b->w_type[i]) continue;
                done[j] = true;
                for (unsigned long t = 0; t < n_tok; ++t)
                    jobs.push_back(MvJob{b->w[j], x + t * E, b->bias[j], outs[j] + t * rows[j], rows[j]});
            }
            if (const int rc = mv_launch_all(c, b->w_type[i], jobs, E, "attn_qkv_chunk")) return rc;
        }
    }
    if (rope_one) {
        const uint64_t nb_q = (n_tok * H + 15) / 16, nb_kv = (n_tok * G + 15) / 16;
        const bool from_sums = qkv_sums.slices >= 2;
        const float *const ps = qkv_sums.part;
        struct Base {
            void *q_out;
            const float *q;
            uint32_t n_heads, q_f16, nb_q;
            void *kp, *vp;
            const float *k, *v;
            const int *pos;
            const uint32_t *pages, *slots;
            uint64_t n_tok;
            uint32_t n_kv_heads;
            uint64_t pt;
            RopeParams r;
            uint32_t *err;
        } a{qdst, from_sums ? ps + qkv_sums.off[0] : q, (uint32_t) H, chunk ? 1u : 0u, (uint32_t) nb_q,
            b->k_pages, b->v_pages, from_sums ? ps + qkv_sums.off[1] : k, from_sums ? ps + qkv_sums.off[2] : v,
            pos, page_ids, slots, n_tok, (uint32_t) G, b->page_tokens,
            rope_params(b->n_rot, b->freq_base, b->freq_scale, b->ext_factor, b->attn_factor, b->corr_lo,
                        b->corr_hi, 1),
            c->err_word};
        // moearc_rope_qkv_sums64_k's parameters: the same, then the biases and the slices
        struct Sums {
            Base base;
            const float *bq, *bk, *bv;
            uint64_t part_stride;
            uint32_t n_slices, pad;
        };
        static_assert(sizeof(Base) % 8 == 0 && offsetof(Sums, bq) == sizeof(Base), "rope_qkv_sums argument layout");
        c->err_armed = true;
        if (from_sums) {
            // slice starts stay 16-byte aligned: every matrix has a multiple of 64 rows
            if (((uintptr_t) a.q | (uintptr_t) a.k | (uintptr_t) a.v) % 16 != 0 || qkv_sums.stride % 4 != 0) return ERR;
            const Sums as{a, b->bias[0], b->bias[1], b->bias[2], qkv_sums.stride, qkv_sums.slices, 0u};
            if (const int rc = launch2d(c, c->f_rope_sums64, (unsigned) (nb_q + nb_kv), 1, 256, as, "rope_qkv_sums", H, D))
                return rc;
        } else if (const int rc = launch2d(c, c->f_rope_qkv64, (unsigned) (nb_q + nb_kv), 1, 256, a, "rope_qkv_chunk",
                                           H, D)) {
            return rc;
        }
    } else {
        if (const int rc = rope_launch(c, chunk ? c->f_rope_f16 : c->f_rope, qdst, q, pos, n_tok, H, D, b->n_rot,
                                       b->freq_base, b->freq_scale, b->ext_factor, b->attn_factor, b->corr_lo,
                                       b->corr_hi, 1))
            return rc;
        if (const int rc = moearc_rope_kv_append_chunk(c, b->k_pages, b->v_pages, k, v, pos, page_ids, slots,
                                                       n_tok, G, D, b->page_tokens, b->n_rot, b->freq_base,
                                                       b->freq_scale, b->ext_factor, b->attn_factor,
                                                       b->corr_lo, b->corr_hi, 1, 1u))
            return rc;
    }
    // With the output projection on the MFMA product (a format without block sums) and the
    // default prefill kernels, the prefill writes the product's f16 hi + lo activation split
    // itself, in place of an f32 output and a split launch (the same halves).
    const bool proj_mm = n_tok >= 2 && mm_check(b->w_type[3], b->w[3], n_tok, E, q_rows) == OK;
    const bool att_split = c->block_fused && proj_mm && !mm_needs_sums(b->w_type[3]) && prefill_is_fast(c, b->scale);
    uint16_t *axh = nullptr, *axl = nullptr;
    float *axs = nullptr;
    if (att_split)
        if (const int rc = mm_split_space(c, nq, &axh, &axl, &axs)) return rc;
    if (n_tok == 1) {  // one decode step: the split-K decode kernel, f32 q (moe.rs:2044-2060)
        const unsigned long n_kv = pos0 + 1, kv_begin = b->n_swa && n_kv > b->n_swa ? n_kv - b->n_swa : 0;
        if (const int rc = moearc_attn_decode(c, att, qr, b->k_pages, b->v_pages, b->block_table, b->sinks, H, G,
                                              D, kv_begin, n_kv, b->page_tokens, b->scale, 1u))
            return rc;
    } else if (const int rc = prefill_launch(c, att_split ? (void *) axh : (void *) att,
                                             att_split ? MOEARC_OUT_F16 : MOEARC_OUT_F32, axl, q16, b->k_pages,
                                             b->v_pages, b->block_table, b->sinks, n_tok, pos0, b->n_swa, H, G,
                                             D, b->page_tokens, b->scale, 1u)) {
        return rc;
    }
    // h += W_o attn (+ bias_o), the residual add folded into the product's store
    (void) proj;
    if (proj_mm) {
        uint16_t *xh = axh, *xl = axl;
        float *xs = axs;
        if (!att_split)
            if (const int rc = mm_split(c, att, nq, &xh, &xl, &xs, mm_needs_sums(b->w_type[3]))) return rc;
        const MmMat mat{b->w[3], b->bias[3], h, E, E};
        return mm_launch(c, b->w_type[3], &mat, 1, xh, xl, xs, n_tok, q_rows, "attn_proj_mm", true);
    }
    std::vector<MvJob> jobs;
    for (unsigned long t = 0; t < n_tok; ++t)
        jobs.push_back(MvJob{b->w[3], att + t * q_rows, b->bias[3], h + t * E, E, true});
    return mv_launch_all(c, b->w_type[3], jobs, q_rows, "attn_proj_chunk");
}
