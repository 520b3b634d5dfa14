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
    hipFunction_t f_rope = nullptr, f_rope_append_chunk = nullptr;
    hipFunction_t f_dec_general = nullptr;
    hipFunction_t f_dec_fast[7] = {};  // KV heads x waves per head: 1x4, 1x16, 2x8, 4x4, 8x2, 1x8, 2x4
    hipFunction_t f_dec_merge = nullptr;
    unsigned merge_threads = 0;  // the merge kernel's launch bound (its work-group size)
    hipFunction_t f_mv[7][4] = {};  // matvec: format (F32 F16 Q8_0 Q4_K Q5_K Q6_K MXFP4) x pieces per lane 1/2/4/8
    hipFunction_t f_add = nullptr;
    hipFunction_t f_mm[6][2] = {}, f_split = nullptr, f_bsums = nullptr;  // Q8_0 F16 Q4_K Q5_K MXFP4 Q6_K x 16 / 32 rows per wave
    uint16_t *mm_ws = nullptr;  // f16 hi / lo split of a chunk's activations
    size_t mm_ws_halves = 0;
    hipFunction_t f_prefill[4] = {};      // group 1, 2, 4, 8
    hipFunction_t f_prefill_precise[4] = {};  // the same with p split into f16 hi + lo
    bool prefill_precise = false;         // MOEARC_PREFILL_PRECISE=1: p split into f16 hi + lo
    bool profiling = false;
    std::vector<Pending> pending;
    std::vector<KernelTime> totals;
    std::vector<hipEvent_t> event_pool;
    // split-K workspace: one partial record per work-group of the split kernel
    float *ws = nullptr;
    size_t ws_floats = 0;
    uint32_t *counters = nullptr;  // fused-merge arrival counters
    size_t counters_n = 0;
    int decode_variant_override = -1;  // MOEARC_DECODE_VARIANT, e.g. "4x4"
    unsigned long split_override = 0;  // MOEARC_DECODE_SPLIT (keys per split)
    float *blk_ws = nullptr;  // attention-block chunk: q, k, v, f16 q, attention output, projection
    size_t blk_ws_bytes = 0;
    unsigned long mv_rpw_override = 0;  // MOEARC_MATVEC_RPW: rows per wave of the matvec launches
    unsigned mv_waves_override = 0;     // MOEARC_MATVEC_WAVES: 4 or 8 waves per work-group
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
    if (!e1) return;
    hipEventRecord(e1, c->stream);
    char key[96];
    std::snprintf(key, sizeof(key), "%s r%lu m%lu", what, r, m);
    c->pending.push_back(Pending{key, start, e1});
    if (c->pending.size() >= 16384) flush_events(c);
}

// Launch `f` with one by-value argument block. With profiling on, a HIP event pair brackets the
// launch under the key "<what> r<r> m<m>" (the reference's key format, kernels.cpp:1905-1916).
template <typename Args>
int launch2d(moearc_ctx *c, hipFunction_t f, unsigned grid, unsigned grid_y, unsigned block,
             const Args &args, const char *what, unsigned long r, unsigned long m,
             unsigned lds_bytes = 0) {
    if (!f) return ERR;
    hipEvent_t e0 = nullptr;
    if (c->profiling && (e0 = take_event(c))) hipEventRecord(e0, c->stream);
    size_t size = sizeof(Args);
    void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, (void *) &args, HIP_LAUNCH_PARAM_BUFFER_SIZE,
                      &size, HIP_LAUNCH_PARAM_END};
    const hipError_t err =
        hipModuleLaunchKernel(f, grid, grid_y, 1, block, 1, 1, lds_bytes, c->stream, nullptr, config);
    if (e0) record_bracket(c, e0, what, r, m);
    return err == hipSuccess ? OK : ERR;
}

template <typename Args>
int launch(moearc_ctx *c, hipFunction_t f, unsigned grid, unsigned block, const Args &args,
           const char *what, unsigned long r, unsigned long m) {
    return launch2d(c, f, grid, 1, block, args, what, r, m);
}

int ensure_workspace(moearc_ctx *c, size_t floats) {
    if (floats <= c->ws_floats) return OK;
    if (c->ws) {
        hipStreamSynchronize(c->stream);  // the previous workspace may still be in use
        hipFree(c->ws);
        c->ws = nullptr;
        c->ws_floats = 0;
    }
    if (hipMalloc((void **) &c->ws, floats * sizeof(float)) != hipSuccess) return ERR;
    c->ws_floats = floats;
    return OK;
}

// Arrival counters of the fused decode merge. Each launch's last work-group per block resets its
// counter, so they only need zeroing when allocated (by the zero kernel, on the stream).
int ensure_counters(moearc_ctx *c, size_t n) {
    if (n <= c->counters_n) return OK;
    if (c->counters) {
        hipStreamSynchronize(c->stream);
        hipFree(c->counters);
        c->counters = nullptr;
        c->counters_n = 0;
    }
    n = std::max<size_t>(n, 1024);
    if (hipMalloc((void **) &c->counters, n * sizeof(uint32_t)) != hipSuccess) return ERR;
    const int rc = moearc_zero(c, (float *) c->counters, n);
    if (rc) return rc;
    c->counters_n = n;
    return OK;
}

// ---- decode dispatch ----------------------------------------------------------------------------

struct SeqSpan {
    uint32_t begin, end;
};

// The split-K kernel masks keys with -inf scores before multiplying by scale*log2(e) and takes
// its running maximum on raw scores, so it needs a positive, finite scale; any other scale runs on
// the general kernel.
bool fast_decode_ok(unsigned long n_heads, unsigned long n_kv_heads, unsigned long head_dim,
                    unsigned long page_tokens, unsigned int kv_type, float scale) {
    return kv_type == 1u && head_dim == 64 && n_heads / n_kv_heads <= 16 && is_pow2(page_tokens) &&
           page_tokens <= (1ul << 30) && scale > 0.f && scale <= 3.0e38f;
}

// Block-table entries the split-K kernel stages in LDS per work-group (PT_CAP in the kernel).
constexpr uint64_t kPageTableCap = 1024;

// Split-K decode variants: KV heads per work-group x waves per KV head (moearc_attn_decode_f16d64_*).
// Split-K decode variants: kb KV heads x wpk waves per work-group (kernel f_dec_fast[kernel]), the
// work-group count the split length aims for, and whether the splits are merged inside the launch
// (by the last work-group of each block to finish) rather than by the merge kernel.
struct DecodeVariant {
    const char *name;
    int kernel;
    unsigned kb, wpk, target_wgs;
    bool fused;
};
constexpr int kNumDecodeVariants = 8;
constexpr DecodeVariant kDecodeVariants[kNumDecodeVariants] = {
    {"1x4", 0, 1, 4, 384, false},  {"1x16", 1, 1, 16, 384, false}, {"2x8", 2, 2, 8, 384, false},
    {"4x4", 3, 4, 4, 384, false},  {"8x2", 4, 8, 2, 384, false},   {"1x4f", 0, 1, 4, 256, true},
    {"1x8", 5, 1, 8, 384, false},  {"2x4", 6, 2, 4, 384, false},
};

// Variant and keys per split. A work-group reads kb*128 bytes of each key row (kb KV heads; four
// keep HBM accesses row-local) with wpk waves per head; the split is sized so that the launch has
// about the variant's target work-group count, rounded up to whole 32-key tiles per wave. Returns
// false when a split would span more pages than the kernel stages.
bool plan_split(moearc_ctx *c, const std::vector<SeqSpan> &spans, unsigned long G,
                unsigned long page_tokens, int &variant, std::vector<uint32_t> &split_len) {
    variant = G >= 4 ? 3 : (G == 2 ? 2 : (G == 1 ? 1 : 3));
    if (c->decode_variant_override >= 0) variant = c->decode_variant_override;
    uint64_t keys = 0;
    for (auto &s : spans) keys += (uint64_t) (s.end - s.begin);
    auto base_of = [&](int v) {
        const uint64_t nkb = (G + kDecodeVariants[v].kb - 1) / kDecodeVariants[v].kb;
        const uint64_t target_wgs = kDecodeVariants[v].target_wgs;
        return (keys * nkb + target_wgs - 1) / target_wgs;
    };
    // Too few keys to give the 4-head work-groups full splits (short contexts, windowed layers):
    // one-head work-groups of 4 waves give 4x the work-groups (measured: 4K keys 12.4 -> 10.4 us,
    // 32 sequences of SWA-128 10.5 -> 7.8 us).
    if (c->decode_variant_override < 0 && variant == 3 && base_of(3) < 32ull * kDecodeVariants[3].wpk)
        variant = 0;
    const unsigned wpk = kDecodeVariants[variant].wpk;
    const uint64_t quantum = 32ull * wpk;  // one tile per wave
    uint64_t base = base_of(variant);
    split_len.resize(spans.size());
    for (size_t i = 0; i < spans.size(); ++i) {
        uint64_t len = c->split_override ? c->split_override : base;
        len = std::max<uint64_t>(len, quantum);
        len = (len + quantum - 1) / quantum * quantum;
        if (len / page_tokens + 2 > kPageTableCap) return false;
        split_len[i] = (uint32_t) std::min<uint64_t>(len, 0x40000000ull);
    }
    return true;
}

int decode_launch_body(moearc_ctx *c, void *out, unsigned int out_f16, const float *q,
                       const void *k_pages, const void *v_pages, const unsigned int *block_tables,
                       unsigned long bt_stride, const std::vector<SeqSpan> &spans,
                       const float *sinks, unsigned long n_heads, unsigned long n_kv_heads,
                       unsigned long head_dim, unsigned long page_tokens, float scale,
                       unsigned int kv_type, size_t nseq, size_t per);

int decode_launch(moearc_ctx *c, void *out, unsigned int out_f16, const float *q,
                  const void *k_pages, const void *v_pages, const unsigned int *block_tables,
                  unsigned long bt_stride, const std::vector<SeqSpan> &spans, const float *sinks,
                  unsigned long n_heads, unsigned long n_kv_heads, unsigned long head_dim,
                  unsigned long page_tokens, float scale, unsigned int kv_type) {
    const size_t nseq = spans.size();
    const size_t per = MOEARC_MAX_SEQS_PER_LAUNCH;
    // With profiling on, the whole call is one bracket under the reference's key; the kernels it
    // launches are also timed under their own keys.
    hipEvent_t call0 = nullptr;
    if (c->profiling && (call0 = take_event(c))) hipEventRecord(call0, c->stream);
    const int rc_all = decode_launch_body(c, out, out_f16, q, k_pages, v_pages, block_tables,
                                          bt_stride, spans, sinks, n_heads, n_kv_heads, head_dim,
                                          page_tokens, scale, kv_type, nseq, per);
    if (call0) record_bracket(c, call0, "attn_decode", n_heads, head_dim);
    return rc_all;
}

int decode_launch_body(moearc_ctx *c, void *out, unsigned int out_f16, const float *q,
                       const void *k_pages, const void *v_pages, const unsigned int *block_tables,
                       unsigned long bt_stride, const std::vector<SeqSpan> &spans,
                       const float *sinks, unsigned long n_heads, unsigned long n_kv_heads,
                       unsigned long head_dim, unsigned long page_tokens, float scale,
                       unsigned int kv_type, size_t nseq, size_t per) {
    const bool fast_shape = fast_decode_ok(n_heads, n_kv_heads, head_dim, page_tokens, kv_type, scale);
    for (size_t s0 = 0; s0 < nseq; s0 += per) {
        const size_t cnt = std::min(per, nseq - s0);
        const float *qb = q + s0 * n_heads * head_dim;
        const size_t out_off = s0 * n_heads * head_dim * (out_f16 ? 2 : 4);
        void *ob = (char *) out + out_off;
        const unsigned int *btb = block_tables + s0 * bt_stride;
        std::vector<SeqSpan> sub(spans.begin() + s0, spans.begin() + s0 + cnt);
        int variant = 3;
        std::vector<uint32_t> split_len;
        const bool fast = fast_shape && plan_split(c, sub, n_kv_heads, page_tokens, variant, split_len);
        if (!fast) {
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
                a.kv_begin[i] = spans[s0 + i].begin;
                a.n_kv[i] = spans[s0 + i].end;
            }
            const int rc = launch(c, c->f_dec_general, (unsigned) (cnt * n_heads), 256, a,
                                  "attn_decode.general", n_heads, head_dim);
            if (rc) return rc;
            continue;
        }
        DecodeArgs a{};
        a.q = qb;
        a.k_pages = (const uint16_t *) k_pages;
        a.v_pages = (const uint16_t *) v_pages;
        a.block_tables = btb;
        a.sinks = sinks;
        a.out = ob;
        a.bt_stride = bt_stride;
        a.n_heads = (uint32_t) n_heads;
        a.n_kv_heads = (uint32_t) n_kv_heads;
        a.group = (uint32_t) (n_heads / n_kv_heads);
        a.pt_shift = log2u(page_tokens);
        a.out_f16 = out_f16;
        a.scale_log2e = scale * 1.4426950408889634f;
        a.n_seqs = (uint32_t) cnt;
        const unsigned kb = kDecodeVariants[variant].kb, wpk = kDecodeVariants[variant].wpk;
        const size_t nkb = (n_kv_heads + kb - 1) / kb;
        a.nkb = (uint32_t) nkb;
        uint32_t items = 0;
        for (size_t i = 0; i < cnt; ++i) {
            a.item_begin[i] = items;
            a.kv_begin[i] = sub[i].begin;
            a.n_kv[i] = sub[i].end;
            a.split_len[i] = split_len[i];
            items += (sub[i].end - sub[i].begin + split_len[i] - 1) / split_len[i];
        }
        for (size_t i = cnt; i <= MOEARC_MAX_SEQS_PER_LAUNCH; ++i) a.item_begin[i] = items;
        const size_t wgs = (size_t) items * nkb;
        if (wgs > 0x7FFFFFFFull) return ERR_ARG;
        if (ensure_workspace(c, (size_t) items * n_kv_heads * MOEARC_PARTIAL_FLOATS)) return ERR;
        a.ws = c->ws;
        const bool any_split = items > cnt;  // some sequence has more than one split
        const bool fused = kDecodeVariants[variant].fused && any_split;
        if (fused) {
            if (ensure_counters(c, cnt * nkb)) return ERR;
            a.counters = c->counters;
        }
        const int rc = launch(c, c->f_dec_fast[kDecodeVariants[variant].kernel], (unsigned) wgs,
                              64u * kb * wpk, a, "attn_decode.split", n_heads, head_dim);
        if (rc) return rc;
        if (any_split && !fused) {
            const int rm = launch2d(c, c->f_dec_merge, (unsigned) (n_heads * MOEARC_MERGE_PARTS), (unsigned) cnt,
                                    c->merge_threads, a, "attn_decode.merge", n_heads, head_dim);
            if (rm) return rm;
        }
    }
    return OK;
}

}  // namespace

extern "C" {

moearc_ctx *moearc_ctx_create(void) {
    auto *c = new moearc_ctx();
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        delete c;
        return nullptr;
    }
    if (hipGetDevice(&c->device) != hipSuccess) {
        delete c;
        return nullptr;
    }
    // Default priority, in-order (the reference's in-order queue, kernels.cpp:806-810).
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return nullptr;
    }
    const char *co_env = std::getenv("MOEARC_CODE_OBJECT");
    const std::string co = co_env ? std::string(co_env) : library_dir() + "/moearc_attn_gfx950.co";
    if (hipModuleLoad(&c->module, co.c_str()) != hipSuccess) {
        std::fprintf(stderr, "moearc: cannot load code object %s\n", co.c_str());
        hipStreamDestroy(c->stream);
        delete c;
        return nullptr;
    }
    struct {
        hipFunction_t *slot;
        const char *name;
    } fns[] = {
        {&c->f_zero, "moearc_zero_k"},
        {&c->f_quant, "moearc_quantize_f16_k"},
        {&c->f_append, "moearc_kv_append_k"},
        {&c->f_append_chunk, "moearc_kv_append_chunk_k"},
        {&c->f_rope, "moearc_rope_k"},
        {&c->f_rope_append_chunk, "moearc_rope_kv_append_chunk_k"},
        {&c->f_dec_general, "moearc_attn_decode_general_k"},
        {&c->f_dec_fast[0], "moearc_attn_decode_f16d64_k1w4"},
        {&c->f_dec_fast[1], "moearc_attn_decode_f16d64_k1w16"},
        {&c->f_dec_fast[2], "moearc_attn_decode_f16d64_k2w8"},
        {&c->f_dec_fast[3], "moearc_attn_decode_f16d64_k4w4"},
        {&c->f_dec_fast[4], "moearc_attn_decode_f16d64_k8w2"},
        {&c->f_dec_fast[5], "moearc_attn_decode_f16d64_k1w8"},
        {&c->f_dec_fast[6], "moearc_attn_decode_f16d64_k2w4"},
        {&c->f_dec_merge, "moearc_attn_decode_merge"},
        {&c->f_add, "moearc_add_k"},
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
        {&c->f_bsums, "moearc_block_sums_k"},
        {&c->f_split, "moearc_split_f16_k"},
    };
    for (auto &f : fns) {
        if (hipModuleGetFunction(f.slot, c->module, f.name) != hipSuccess) {
            std::fprintf(stderr, "moearc: code object %s lacks kernel %s\n", co.c_str(), f.name);
            hipModuleUnload(c->module);
            hipStreamDestroy(c->stream);
            delete c;
            return nullptr;
        }
    }
    int merge_threads = 0;
    if (hipFuncGetAttribute(&merge_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->f_dec_merge) !=
            hipSuccess || merge_threads != MOEARC_MERGE_THREADS) {
        std::fprintf(stderr, "moearc: cannot read the merge kernel's work-group size\n");
        hipModuleUnload(c->module);
        hipStreamDestroy(c->stream);
        delete c;
        return nullptr;
    }
    c->merge_threads = (unsigned) merge_threads;
    if (const char *pp = std::getenv("MOEARC_PREFILL_PRECISE")) c->prefill_precise = pp[0] == '1';
    for (int i = 0; i < 8; ++i) {
        const bool precise = i >= 4;
        char name[64];
        std::snprintf(name, sizeof(name), "moearc_attn_prefill_%sg%d", precise ? "precise_" : "", 1 << (i & 3));
        hipFunction_t *slot = precise ? &c->f_prefill_precise[i & 3] : &c->f_prefill[i & 3];
        if (hipModuleGetFunction(slot, c->module, name) != hipSuccess) {
            std::fprintf(stderr, "moearc: code object %s lacks kernel %s\n", co.c_str(), name);
            hipModuleUnload(c->module);
            hipStreamDestroy(c->stream);
            delete c;
            return nullptr;
        }
    }
    for (int t = 0; t < 7; ++t) {
        for (int i = 0; i < 4; ++i) {
            if ((1u << i) > moearc_mv_ppl_max(kMvTypes[t])) continue;
            char name[64];
            std::snprintf(name, sizeof(name), "moearc_matvec_%s_p%u", kMvNames[t], 1u << i);
            if (hipModuleGetFunction(&c->f_mv[t][i], c->module, name) != hipSuccess) {
                std::fprintf(stderr, "moearc: code object %s lacks kernel %s\n", co.c_str(), name);
                hipModuleUnload(c->module);
                hipStreamDestroy(c->stream);
                delete c;
                return nullptr;
            }
        }
    }
    if (const char *r = std::getenv("MOEARC_MATVEC_RPW")) c->mv_rpw_override = std::strtoul(r, nullptr, 10);
    if (const char *w = std::getenv("MOEARC_MATVEC_WAVES")) {
        const unsigned long v = std::strtoul(w, nullptr, 10);
        if (v == 4 || v == 8) c->mv_waves_override = (unsigned) v;
    }
    const char *ev = std::getenv("MOEARC_PROFILE_EVENTS");
    c->profiling = ev && ev[0] == '1';
    if (const char *w = std::getenv("MOEARC_DECODE_VARIANT")) {
        for (int i = 0; i < kNumDecodeVariants; ++i)
            if (std::strcmp(w, kDecodeVariants[i].name) == 0) c->decode_variant_override = i;
    }
    if (const char *s = std::getenv("MOEARC_DECODE_SPLIT")) c->split_override = std::strtoul(s, nullptr, 10);
    return c;
}

void moearc_ctx_destroy(moearc_ctx *c) {
    if (!c) return;
    hipStreamSynchronize(c->stream);
    for (auto &p : c->pending) {
        hipEventDestroy(p.start);
        hipEventDestroy(p.stop);
    }
    for (auto e : c->event_pool) hipEventDestroy(e);
    if (c->ws) hipFree(c->ws);
    if (c->counters) hipFree(c->counters);
    if (c->blk_ws) hipFree(c->blk_ws);
    if (c->mm_ws) hipFree(c->mm_ws);
    if (c->module) hipModuleUnload(c->module);
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
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

int moearc_rope(moearc_ctx *c, float *dst, const float *src, const int *pos,
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
        float *dst;
        const float *src;
        const int *pos;
        uint64_t n_tokens;
        uint32_t n_heads, head_dim;
        RopeParams r;
    } a{dst, src, pos, n_tokens, (uint32_t) n_heads, (uint32_t) head_dim,
        rope_params(n_dims, freq_base, freq_scale, ext_factor, attn_factor, corr_lo, corr_hi, neox)};
    return launch2d(c, c->f_rope, (unsigned) ((threads + 255) / 256), (unsigned) groups, 256, a,
                    "rope", n_heads, head_dim);
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
    } a{k_pages, v_pages, k, v, pos, page_ids, slots, n_tok, (uint32_t) n_kv_heads,
        (uint32_t) head_dim, page_tokens, kv_type,
        rope_params(n_dims, freq_base, freq_scale, ext_factor, attn_factor, corr_lo, corr_hi, neox)};
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
    return hipStreamSynchronize(c->stream) == hipSuccess ? OK : ERR;
}

int moearc_zero(moearc_ctx *c, float *dst, unsigned long n) {
    if (!c || !dst) return ERR;
    if (n == 0) return OK;
    const unsigned grid = (unsigned) std::min<unsigned long>((n + 255) / 256, 65536ul);
    struct {
        float *d;
        uint64_t n;
    } a{dst, n};
    return launch(c, c->f_zero, grid, 256, a, "zero", n, 0);
}

int moearc_device_name(moearc_ctx *c, char *out, unsigned long cap) {
    if (!c || !out || cap == 0) return ERR;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, c->device) != hipSuccess) return ERR;
    std::snprintf(out, cap, "%s (%s)", p.name, p.gcnArchName);
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
    hipStreamSynchronize(c->stream);
    hipFree(p);
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
    char key[48];
    std::snprintf(key, sizeof(key), "%s %s", what, kMvKeys[t]);
    return launch2d(c, c->f_mv[t][li], (unsigned) wgs, 1, 64u * waves, a, key, key_r, key_m,
                    (unsigned) (x_bytes + (uint64_t) waves * wave_buf));
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
    return mv_launch(c, 0, &j, 1, n_cols, "mvf32", n_rows, 1);
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
    return launch(c, c->f_add, grid, 256, args, "add", n, 0);
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
    return launch(c, c->f_quant, grid, 256, a, "quantize_f16", n, 0);
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
    return launch(c, c->f_append, (unsigned) ((row + 255) / 256), 256, a, "kv_append", n_kv_heads,
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
    } a{k_pages, v_pages, k, v, page_ids, slots, n_tok, row, page_tokens, kv_type};
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
    std::vector<SeqSpan> spans{SeqSpan{(uint32_t) kv_begin, (uint32_t) n_kv}};
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
    std::vector<SeqSpan> spans(n_seqs);
    for (unsigned long b = 0; b < n_seqs; ++b) {
        if (n_kv[b] == 0 || kv_begin[b] >= n_kv[b]) return ERR_ARG;
        if ((n_kv[b] + page_tokens - 1) / page_tokens > bt_stride) return ERR_ARG;
        spans[b] = SeqSpan{kv_begin[b], n_kv[b]};
    }
    return decode_launch(c, out, out_type, q, k_pages, v_pages, block_tables, bt_stride, spans,
                         sinks, n_heads, n_kv_heads, head_dim, page_tokens, scale, kv_type);
}

int moearc_attn_prefill(moearc_ctx *c, void *out, unsigned int out_type, const void *q,
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
    // The single-f16 kernels pre-scale Q by scale*log2(e) in f16, which stays in range for
    // |scale*log2(e)| <= 1 (every softmax scale up to 0.69); larger scales take the precise kernels.
    const float scale_log2e = scale * 1.4426950408889634f;
    const bool precise = c->prefill_precise || !(std::fabs(scale_log2e) <= 1.0f);
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
    const uint64_t wgs = (uint64_t) a.n_qtiles * n_kv_heads;
    if (wgs > 0x7FFFFFFFull) return ERR_ARG;
    return launch(c, f, (unsigned) wgs, MOEARC_PREFILL_THREADS, a, "attn_prefill",
                  n_heads, head_dim);
}

}  // extern "C"

namespace {

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

// y = W x over a chunk, x given as its f16 split (xh, xl) of n_tok x n_cols.
int mm_launch(moearc_ctx *c, unsigned ty, float *y, unsigned long y_stride, const void *w,
              const uint16_t *xh, const uint16_t *xl, const float *xs, const float *bias, unsigned long n_tok,
              unsigned long n_rows, unsigned long n_cols, const char *what, bool accumulate = false) {
    MatmulArgs a{};
    a.accumulate = accumulate ? 1u : 0u;
    a.w = static_cast<const uint8_t *>(w);
    a.xh = xh;
    a.xl = xl;
    a.xs = xs;
    a.bias = bias;
    a.y = y;
    a.row_bytes = (uint64_t) n_cols / moearc_mv_be(ty) * moearc_mv_bb(ty);
    a.rows = (uint32_t) n_rows;
    a.cols = (uint32_t) n_cols;
    a.n_tok = (uint32_t) n_tok;
    a.y_stride = (uint32_t) y_stride;
    // 32 rows per wave halves the activation loads per MFMA, but only pays while the launch still
    // has about two work-groups per CU; shorter chunks take 16 rows per wave.
    const unsigned long tok_groups = (n_tok + MOEARC_MM_TOKENS - 1) / MOEARC_MM_TOKENS;
    const int r2 = ((n_rows + 127) / 128) * tok_groups >= 512 ? 1 : 0;
    const unsigned long rows_per_wg = r2 ? 128 : 64;
    return launch2d(c, c->f_mm[mm_index(ty)][r2], (unsigned) ((n_rows + rows_per_wg - 1) / rows_per_wg),
                    (unsigned) tok_groups, 256, a, what, n_rows, n_tok);
}

// The f16 hi / lo split of x (n floats, n a multiple of 32) and its 32-element block sums into
// the context's buffer.
int mm_split(moearc_ctx *c, const float *x, size_t n, uint16_t **xh, uint16_t **xl, float **xs) {
    const size_t halves = 2 * n + n / 16;  // hi, lo, then n / 32 floats
    if (halves > c->mm_ws_halves) {
        if (c->mm_ws) {
            hipStreamSynchronize(c->stream);
            hipFree(c->mm_ws);
            c->mm_ws = nullptr;
            c->mm_ws_halves = 0;
        }
        if (hipMalloc((void **) &c->mm_ws, halves * sizeof(uint16_t)) != hipSuccess) return ERR;
        c->mm_ws_halves = halves;
    }
    *xh = c->mm_ws;
    *xl = c->mm_ws + n;
    *xs = (float *) (c->mm_ws + 2 * n);  // 4-byte aligned: n is a multiple of 32
    struct {
        const float *x;
        float *xs;
        uint64_t n;
    } bs{x, *xs, n / 32};
    if (const int rc = launch(c, c->f_bsums, (unsigned) std::min<size_t>((n / 32 + 255) / 256, 65536), 256, bs,
                              "block_sums", n / 32, 0))
        return rc;
    struct {
        const float *x;
        uint16_t *hi, *lo;
        uint64_t n;
    } a{x, *xh, *xl, n};
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
    if (const int rc = mm_split(c, x, n_tok * n_cols, &xh, &xl, &xs)) return rc;
    return mm_launch(c, type_id, y, n_rows, w, xh, xl, xs, bias, n_tok, n_rows, n_cols, "matmul");
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

    // working memory: q, k, v, rotated q, f16 q, attention output, projection
    const size_t nq = n_tok * q_rows, nkv = n_tok * kv_rows;
    const size_t floats = nq + 2 * nkv + nq + (nq + 1) / 2 + nq + n_tok * E;
    if (floats * sizeof(float) > c->blk_ws_bytes) {
        if (c->blk_ws) {
            hipStreamSynchronize(c->stream);
            hipFree(c->blk_ws);
            c->blk_ws = nullptr;
            c->blk_ws_bytes = 0;
        }
        if (hipMalloc((void **) &c->blk_ws, floats * sizeof(float)) != hipSuccess) return ERR;
        c->blk_ws_bytes = floats * sizeof(float);
    }
    float *q = c->blk_ws, *k = q + nq, *v = k + nkv, *qr = v + nkv;
    uint16_t *q16 = (uint16_t *) (qr + nq);
    float *att = qr + nq + (nq + 1) / 2, *proj = att + nq;

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
        if (const int rc = mm_split(c, x, n_tok * E, &xh, &xl, &xs)) return rc;
        float *outs[3] = {q, k, v};
        const unsigned long rows[3] = {q_rows, kv_rows, kv_rows};
        for (int i = 0; i < 3; ++i)
            if (const int rc = mm_launch(c, b->w_type[i], outs[i], rows[i], b->w[i], xh, xl, xs, b->bias[i], n_tok,
                                         rows[i], E, "attn_qkv_mm"))
                return rc;
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
    // RoPE of q (narrowed to f16 for the prefill kernel when there is a chunk); RoPE of K fused
    // with the K/V append
    if (const int rc = moearc_rope(c, qr, q, pos, n_tok, H, D, b->n_rot, b->freq_base, b->freq_scale,
                                   b->ext_factor, b->attn_factor, b->corr_lo, b->corr_hi, 1))
        return rc;
    if (n_tok > 1)
        if (const int rc = moearc_quantize_f16(c, q16, qr, nq)) return rc;
    if (const int rc = moearc_rope_kv_append_chunk(c, b->k_pages, b->v_pages, k, v, pos, page_ids, slots,
                                                   n_tok, G, D, b->page_tokens, b->n_rot, b->freq_base,
                                                   b->freq_scale, b->ext_factor, b->attn_factor,
                                                   b->corr_lo, b->corr_hi, 1, 1u))
        return rc;
    if (n_tok == 1) {  // one decode step: the split-K decode kernel, f32 q (moe.rs:2044-2060)
        const unsigned long n_kv = pos0 + 1, kv_begin = b->n_swa && n_kv > b->n_swa ? n_kv - b->n_swa : 0;
        if (const int rc = moearc_attn_decode(c, att, qr, b->k_pages, b->v_pages, b->block_table, b->sinks, H, G,
                                              D, kv_begin, n_kv, b->page_tokens, b->scale, 1u))
            return rc;
    } else if (const int rc = moearc_attn_prefill(c, att, MOEARC_OUT_F32, q16, b->k_pages, b->v_pages,
                                                  b->block_table, b->sinks, n_tok, pos0, b->n_swa, H, G, D,
                                                  b->page_tokens, b->scale, 1u)) {
        return rc;
    }
    // h += W_o attn (+ bias_o), the residual add folded into the product's store
    (void) proj;
    if (n_tok >= 2 && mm_check(b->w_type[3], b->w[3], n_tok, E, q_rows) == OK) {
        uint16_t *xh, *xl;
        float *xs;
        if (const int rc = mm_split(c, att, nq, &xh, &xl, &xs)) return rc;
        return mm_launch(c, b->w_type[3], h, E, b->w[3], xh, xl, xs, b->bias[3], n_tok, E, q_rows, "attn_proj_mm",
                         true);
    }
    std::vector<MvJob> jobs;
    for (unsigned long t = 0; t < n_tok; ++t)
        jobs.push_back(MvJob{b->w[3], att + t * q_rows, b->bias[3], h + t * E, E, true});
    return mv_launch_all(c, b->w_type[3], jobs, q_rows, "attn_proj_chunk");
}
