// Split-K single-query paged attention for f16 KV with head_dim 64 (the gpt-oss shape: 64 query
// heads over 8 KV heads), on gfx950 MFMA.
//
// Semantics are moearc_attn_decode's (kernels.cpp:1837-1919): for each query head,
//     out = sum_j e^(s_j - M) V_j / (e^(sink - M) + sum_j e^(s_j - M)),  s_j = scale * q.K_j,
// over the span [kv_begin, n_kv) read through the block table.
//
// Work decomposition. A work-group of WAVES wavefronts owns one KV head of one split (a run of
// split_len consecutive keys) of one sequence, and serves every query head of that KV head's group
// from a single read of each K/V row -- the KV bytes cross HBM once, not once per query head. Each
// wave takes 32-key tiles round-robin and keeps its own online-softmax state; the waves merge in
// LDS. A sequence whose span fits one split is finished there (sink applied, output written);
// otherwise each work-group writes a partial record (per-head max, denominator and unnormalised
// output) with agent-coherent (sc1) stores. With an arrival counter per (sequence, KV-head block)
// the last work-group to finish a block merges its splits inside the same launch (the fused
// variant, few splits per block); otherwise moearc_attn_decode_merge, the next launch on the
// stream, combines them.
//
// Per 32-key tile (one wave), all operands in registers, no LDS:
//   loads   K and V rows go from HBM straight into MFMA A-operand layout: lane (g, m) loads 16
//           bytes, channels 8g..8g+7 (and 32+8g..) of key 16*blk + m. Eight 16-byte loads per lane
//           per tile; the next tile's loads are always in flight while this one is computed.
//   QK^T    S^T[32 keys x 16 heads] = K . Q^T, 2 key blocks x 2 channel halves of
//           v_mfma_f32_16x16x32_f16. Q is split q = q_hi + q_lo into two f16 operands (after an
//           exact power-of-two normalisation), so the products see q to ~22 bits; K is exact f16.
//   softmax lane (g, n) holds head n's scores for keys 16*blk + 4g + r. exp2 with scale*log2(e)
//           folded into one multiplier; running max across the four lanes of a head.
//   V^T     the P.V product needs V with keys along the MFMA reduction axis. Multiplying the
//           natural-layout V block by a 0/1 selection matrix on the MFMA unit returns it in the
//           accumulator layout -- lane (g, n) gets channel n of keys 4g..4g+3 -- which is exactly
//           the A-operand layout P.V needs. Exact: each output is one f16 value times 1 plus zeros.
//   P.V     O^T[64 x 16] += V^T[64 x 32] . P^T[32 x 16], P^T straight from the softmax registers,
//           split p = p_hi + p_lo like q.
// Heads beyond the group (columns 8..15 when the group is 8) are computed and discarded: MFMA
// time is not the bound here, HBM is.
#include "common.h"

// Scores live in the log2 domain, x = scale * log2(e) * q.K. Probabilities enter the f16 MFMA
// operands as p * 2^LOG2_PSCALE relative to a per-head reference max m_ref that is only moved
// when a tile's max exceeds it by more than RESCALE_SLACK (the running sums are then rescaled
// once); so p * 2^7 <= 2^(7 + 8) = 32768 stays inside f16, and p_lo (the f16 residual of p_hi)
// stays a normal f16 down to p ~ 2^-10 of the reference, with a 2^-31 floor below that.
#define LOG2_PSCALE 7.0f
#define RESCALE_SLACK 8.0f
#define PT_CAP 1024       // block-table entries one work-group stages in LDS

__device__ __forceinline__ float4_t mfma16(const half8_t a, const half8_t b, const float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8_t as_half8(const u32x4_t v) { return __builtin_bit_cast(half8_t, v); }

__device__ __forceinline__ float wave_max_16_32(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

struct TileRegs {
    u32x4_t k[2][2];  // [key block][channel half], A-operand layout
    u32x4_t v[2][2];
};

// Physical row of logical key j: page table staged in LDS for this work-group's split.
__device__ __forceinline__ uint32_t key_row(const uint32_t *pt_lds, uint32_t j, uint32_t page0,
                                            uint32_t sh) {
    return (pt_lds[(j >> sh) - page0] << sh) | (j & ((1u << sh) - 1u));
}

// Loads one 32-key tile; row_of(j) is the physical row of logical key j (through the page table
// staged in LDS, or straight from the block table).
template <typename RowOf>
__device__ __forceinline__ void load_tile_rows(TileRegs &r, const DecodeArgs &a, RowOf row_of,
                                               uint32_t j0, uint32_t te, uint32_t kvh, uint32_t lane) {
    const uint64_t row_elems = (uint64_t) a.n_kv_heads * 64u;
    const uint32_t g = lane >> 4, m = lane & 15u;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        const uint32_t j = min(j0 + 16u * blk + m, te - 1u);
        const uint64_t off = (uint64_t) row_of(j) * row_elems + (uint64_t) kvh * 64u + 8u * g;
        const uint16_t *ks = a.k_pages + off;
        const uint16_t *vs = a.v_pages + off;
        // Plain loads: the non-temporal hint measured 15% slower for this pattern (each 128-byte
        // line is consumed by two 64-byte requests, which the hint lets the L2 evict in between).
        r.k[blk][0] = *(const u32x4_t *) ks;
        r.k[blk][1] = *(const u32x4_t *) (ks + 32);
        r.v[blk][0] = *(const u32x4_t *) vs;
        r.v[blk][1] = *(const u32x4_t *) (vs + 32);
    }
}

__device__ __forceinline__ void load_tile(TileRegs &r, const DecodeArgs &a, const uint32_t *pt_lds,
                                          uint32_t page0, uint32_t j0, uint32_t te, uint32_t kvh,
                                          uint32_t lane) {
    const uint32_t sh = a.pt_shift;
    load_tile_rows(r, a, [&](uint32_t j) { return key_row(pt_lds, j, page0, sh); }, j0, te, kvh, lane);
}

// The same tile with its page ids read from the block table in global memory: a wave's first tile
// issues its loads one round trip after launch instead of after the LDS staging and its barrier.
__device__ __forceinline__ void load_tile_bt(TileRegs &r, const DecodeArgs &a, const uint32_t *bt,
                                             uint32_t j0, uint32_t te, uint32_t kvh, uint32_t lane) {
    const uint32_t sh = a.pt_shift;
    load_tile_rows(r, a, [&](uint32_t j) { return (bt[j >> sh] << sh) | (j & ((1u << sh) - 1u)); },
                   j0, te, kvh, lane);
}

struct SoftmaxState {
    float m;        // reference max (log2 domain), uniform over the 4 lanes of a head
    float l;        // running denominator in the m-frame, partial over this lane's keys
    float4_t O[4];  // O^T[16*mb + 4g + r][n] in the m-frame
};

__device__ __forceinline__ void process_tile(SoftmaxState &st, const TileRegs &r,
                                             const half8_t (&qhi)[2], const half8_t (&qlo)[2],
                                             const half8_t (&sel)[2], float c, uint32_t j0,
                                             uint32_t te, uint32_t g) {
    // QK^T: S[blk] lane (g, n) reg i = raw score of key j0 + 16*blk + 4g + i for head n
    float4_t S[2];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        float4_t s = (float4_t){0.f, 0.f, 0.f, 0.f};
        s = mfma16(as_half8(r.k[blk][0]), qhi[0], s);
        s = mfma16(as_half8(r.k[blk][0]), qlo[0], s);
        s = mfma16(as_half8(r.k[blk][1]), qhi[1], s);
        s = mfma16(as_half8(r.k[blk][1]), qlo[1], s);
        S[blk] = s;
    }
    if (j0 + 32u > te) {  // the span's last, partial tile (uniform branch)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (j0 + 16u * (i >> 2) + 4u * g + (i & 3) >= te) S[i >> 2][i & 3] = -INFINITY;
    }
    float tmax = fmaxf(fmaxf(fmaxf(S[0][0], S[0][1]), fmaxf(S[0][2], S[0][3])),
                       fmaxf(fmaxf(S[1][0], S[1][1]), fmaxf(S[1][2], S[1][3])));
    tmax = wave_max_16_32(tmax) * c;
    // Move the reference only when some head's max outgrew it by more than the slack.
    if (__builtin_amdgcn_ballot_w64(tmax > st.m + RESCALE_SLACK) != 0) {
        const float m_new = fmaxf(st.m, tmax);
        const float corr = exp2_fast(st.m - m_new);  // first tile: exp2(-inf) = 0
        st.m = m_new;
        st.l *= corr;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) st.O[mb] *= corr;
    }
    const float bias = LOG2_PSCALE - st.m;
    half8_t phi, plo;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float ps = exp2_fast(fmaf(S[i >> 2][i & 3], c, bias));
        psum += ps;
        const _Float16 hi = (_Float16) ps;
        phi[i] = hi;
        plo[i] = (_Float16) (ps - (float) hi);
    }
    st.l += psum;
    // V^T via the selection product, then P.V, one 16-channel block at a time
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
        const int hf = mb >> 1, sl = mb & 1;
        const float4_t z = (float4_t){0.f, 0.f, 0.f, 0.f};
        const float4_t t0 = mfma16(as_half8(r.v[0][hf]), sel[sl], z);  // keys 4g+i
        const float4_t t1 = mfma16(as_half8(r.v[1][hf]), sel[sl], z);  // keys 16+4g+i
        half8_t va;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            va[i] = (_Float16) t0[i];
            va[4 + i] = (_Float16) t1[i];
        }
        st.O[mb] = mfma16(va, phi, st.O[mb]);
        st.O[mb] = mfma16(va, plo, st.O[mb]);
    }
}

// Agent-scope relaxed atomics on the partial records: global_store/load with sc1, coherent across
// XCDs without an L2 write-back or invalidate.
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store((uint32_t *) p, __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
    return __builtin_bit_cast(float, __hip_atomic_load((uint32_t *) p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Final normalisation with the sink (kernels.cpp:1864-1880), in the log2 domain and the m-frame:
// out = O 2^(M-Mt) / (L 2^(M-Mt) + 2^(sink*log2e - Mt + LOG2_PSCALE)), Mt = max(M, sink*log2e).
__device__ __forceinline__ void write_output(const DecodeArgs &a, uint32_t b, uint32_t hh,
                                             uint32_t d, float M, float L, float acc) {
    const float sink2 = a.sinks ? a.sinks[hh] * MOEARC_LOG2E : -INFINITY;
    const float Mt = fmaxf(M, sink2);
    const float fm = exp2_fast(M - Mt);
    const float den = L * fm + exp2_fast(sink2 - Mt + LOG2_PSCALE);
    const float r = acc * fm / den;
    const uint64_t o = ((uint64_t) b * a.n_heads + hh) * 64u + d;
    if (a.out_f16) ((_Float16 *) a.out)[o] = (_Float16) r;
    else ((float *) a.out)[o] = r;
}

// One work-group: KB consecutive KV heads x WPK waves per KV head, over one split of one
// sequence. Reading KB*128 bytes of every key row per work-group (rather than one 128-byte KV-head
// stripe) keeps HBM accesses row-local; WPK waves per head give enough loads in flight.
template <int KB, int WPK>
__device__ __forceinline__ void decode_body(const DecodeArgs &a) {
    constexpr int WAVES = KB * WPK;
    __shared__ float o_lds[WAVES][16 * 64];
    __shared__ float m_lds[WAVES][16];
    __shared__ float l_lds[WAVES][16];
    __shared__ uint32_t pt_lds[PT_CAP];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t G = a.n_kv_heads;
    const uint32_t nkb = a.nkb;
    const uint32_t kbi = blockIdx.x % nkb;
    const uint32_t item = blockIdx.x / nkb;
    // Sequence 0's span is read unconditionally, with no load depending on another, so a
    // single-sequence launch resolves it in one round trip; later sequences search on.
    uint32_t ib = a.item_begin[0], next = a.item_begin[1], kvb = a.kv_begin[0];
    uint32_t nkv = a.n_kv[0], slen = a.split_len[0];
    // Pin these (and the fields the first loads address with) in SGPRs here: otherwise the compiler
    // folds the sequence-0 reads into the general lookup after its branch, a second round trip.
    asm volatile("" ::"s"(ib), "s"(next), "s"(kvb), "s"(nkv), "s"(slen), "s"(a.pt_shift),
                 "s"(a.n_kv_heads), "s"(a.bt_stride), "s"(a.block_tables), "s"(a.k_pages),
                 "s"(a.v_pages));
    uint32_t b = 0;
    if (item >= next) {
        do ++b; while (item >= a.item_begin[b + 1]);
        ib = a.item_begin[b];
        next = a.item_begin[b + 1];
        kvb = a.kv_begin[b];
        nkv = a.n_kv[b];
        slen = a.split_len[b];
    }
    const uint32_t split = item - ib;
    const uint32_t nsplit = next - ib;
    const uint32_t tb = kvb + split * slen;
    const uint32_t te = min(nkv, tb + slen);
    const uint32_t ntiles = (te - tb + 31u) >> 5;
    const uint32_t kl = wave % KB, sub = wave / KB;
    const uint32_t kvh = kbi * KB + kl;
    const bool kvh_ok = kvh < G;
    const uint32_t group = a.group;
    const uint32_t g = lane >> 4, n = lane & 15u;
    const bool head_ok = kvh_ok && n < group;
    const uint32_t h = min(kvh, G - 1u) * group + (n < group ? n : 0u);
    const uint32_t *bt = a.block_tables + (uint64_t) b * a.bt_stride;
    const bool has_tiles = kvh_ok && sub < ntiles;

    // ---- stage this split's block-table entries in LDS ------------------------------------------
    const uint32_t sh = a.pt_shift;
    const uint32_t page0 = tb >> sh;
    const uint32_t npages = ((te - 1u) >> sh) - page0 + 1u;  // host guarantees <= PT_CAP
    // Start-up order: the page-table and q loads issue first, then this wave's first tile (page
    // ids read straight from the block table), and only then do the page-table stores and the q
    // arithmetic wait for their loads -- so the first KV loads leave one round trip after launch,
    // not after the LDS staging and its barrier.
    constexpr uint32_t PT_PER_THREAD = (PT_CAP + 64u * WAVES - 1u) / (64u * WAVES);
    uint32_t ptv[PT_PER_THREAD];
#pragma unroll
    for (uint32_t k = 0; k < PT_PER_THREAD; ++k) {
        const uint32_t i = threadIdx.x + k * 64u * WAVES;
        ptv[k] = i < npages ? bt[page0 + i] : 0u;
    }

    // ---- Q operands (B of QK^T): lane (g, n) holds head n, channels 32*hf + 8g .. +7 ----------
    float qv[16];
    {
        const float *qrow = a.q + ((uint64_t) b * a.n_heads + h) * 64u;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const float4_t x0 = *(const float4_t *) (qrow + 32 * hf + 8 * g);
            const float4_t x1 = *(const float4_t *) (qrow + 32 * hf + 8 * g + 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qv[8 * hf + i] = head_ok ? x0[i] : 0.f;
                qv[8 * hf + 4 + i] = head_ok ? x1[i] : 0.f;
            }
        }
    }
    // This wave's first tile. Issued unconditionally (a wave without tiles loads an in-span key of
    // an existing KV head and ignores it): a branch here would make the compiler's wait counts at
    // the join assume these loads may be missing and drain them before the q arithmetic.
    TileRegs r0;
    load_tile_bt(r0, a, bt, tb + 32u * sub, te, min(kvh, G - 1u), lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t k = 0; k < PT_PER_THREAD; ++k) {
        const uint32_t i = threadIdx.x + k * 64u * WAVES;
        if (i < npages) pt_lds[i] = ptv[k];
    }

    // Normalise each head's q by a power of two (exact) so that the hi/lo split keeps full relative
    // precision whatever q's magnitude; the inverse power folds into the score multiplier.
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(qv[i]));
    amax = wave_max_16_32(amax);
    int qexp = 0;
    if (amax > 0.f && amax < INFINITY) (void) frexpf(amax, &qexp);
    const float c = ldexpf(a.scale_log2e, qexp - 1);  // score multiplier in the log2 domain
    half8_t qhi[2], qlo[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = ldexpf(qv[8 * hf + i], 1 - qexp);
            const _Float16 hi = (_Float16) x;
            qhi[hf][i] = hi;
            qlo[hf][i] = (_Float16) (x - (float) hi);
        }
    // Selection operands: sel[s] lane (g, n) item i = 1 where 8g + i == 16s + n.
    half8_t sel[2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) sel[s][i] = (8u * g + i == 16u * s + n) ? (_Float16) 1.0f : (_Float16) 0.0f;

    __syncthreads();  // page table ready

    // ---- key loop: wave `sub` of this KV head takes tiles sub, sub + WPK, ... ------------------
    SoftmaxState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) st.O[mb] = (float4_t){0.f, 0.f, 0.f, 0.f};
    if (has_tiles) {
        if constexpr (WAVES <= 8) {
            // Two tiles in flight per wave: the loads of the next tile issue before this one is
            // computed, over two register sets (ra, rb). The wave walks its tiles in pairs with a
            // single loop exit, so every wait leaves exactly the younger set's eight loads
            // outstanding; a pair's second tile past the span (odd tile count) computes nothing
            // (all its keys are at or beyond te, so every weight is zero) and its loads repeat a
            // tile of the span (cache hits).
            const uint32_t nt = (ntiles - sub + WPK - 1u) / WPK;  // this wave's tiles, >= 1
            const uint32_t last = sub + (nt - 1u) * WPK;
            auto tile_of = [&](uint32_t i) { return sub + i * WPK; };
            TileRegs ra = r0, rb;
            for (uint32_t i = 0; i < nt; i += 2) {
                load_tile(rb, a, pt_lds, page0, tb + 32u * min(tile_of(i + 1u), last), te, kvh, lane);
                __builtin_amdgcn_sched_barrier(0);
                process_tile(st, ra, qhi, qlo, sel, c, tb + 32u * tile_of(i), te, g);
                load_tile(ra, a, pt_lds, page0, tb + 32u * min(tile_of(i + 2u), last), te, kvh, lane);
                __builtin_amdgcn_sched_barrier(0);
                process_tile(st, rb, qhi, qlo, sel, c, min(tb + 32u * tile_of(i + 1u), te), te, g);
            }
        } else {
            // 16-wave work-groups (128 VGPRs per wave): one tile in flight per wave, the
            // residency of four waves per SIMD keeps HBM busy.
            process_tile(st, r0, qhi, qlo, sel, c, tb + 32u * sub, te, g);
            for (uint32_t t = sub + WPK; t < ntiles; t += WPK) {
                const uint32_t j0 = tb + 32u * t;
                TileRegs r;
                load_tile(r, a, pt_lds, page0, j0, te, kvh, lane);
                // All eight loads issue before any compute: left alone, the scheduler sinks the V
                // loads below the QK^T MFMAs and every tile pays two memory latencies.
                __builtin_amdgcn_sched_barrier(0);
                process_tile(st, r, qhi, qlo, sel, c, j0, te, g);
            }
        }
    }

    // ---- merge the WPK waves of each KV head in LDS ---------------------------------------------
    float l_run = st.l;
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (head_ok) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
            *(float4_t *) (&o_lds[wave][n * 64u + 16u * mb + 4u * g]) = st.O[mb];
    }
    if (g == 0) {
        m_lds[wave][n] = head_ok ? st.m : -INFINITY;
        l_lds[wave][n] = head_ok ? l_run : 0.f;
    }
    __syncthreads();

    // Threads take (KV head of the block, output element) pairs.
    const uint32_t n_out = group * 64u;
    const bool single = nsplit == 1u;
    for (uint32_t idx = threadIdx.x; idx < KB * n_out; idx += 64u * WAVES) {
        const uint32_t k2 = idx / n_out, e = idx - k2 * n_out;
        const uint32_t kv2 = kbi * KB + k2;
        if (kv2 >= G) break;
        const uint32_t hn = e >> 6, d = e & 63u;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WPK; ++w) M = fmaxf(M, m_lds[w * KB + k2][hn]);
        float L = 0.f, acc = 0.f;
#pragma unroll
        for (int w = 0; w < WPK; ++w) {
            const uint32_t ww = w * KB + k2;
            const float f = exp2_fast(m_lds[ww][hn] - M);  // a wave without tiles has m = -inf: f = 0
            L += l_lds[ww][hn] * f;
            acc += o_lds[ww][hn * 64u + d] * f;
        }
        if (single) {
            write_output(a, b, kv2 * group + hn, d, M, L, acc);
        } else {
            float *rec = a.ws + ((uint64_t) item * G + kv2) * MOEARC_PARTIAL_FLOATS;
            st_agent(rec + 32u + e, acc);
            if (d == 0) {
                st_agent(rec + hn, M);
                st_agent(rec + 16u + hn, L);
            }
        }
    }
    if (single || a.counters == nullptr) return;

    // ---- fused merge: the last work-group of this (sequence, KV-head block) to arrive merges it --
    // Every thread's record stores are complete at agent scope (sc1, waited for) before the arrival
    // is counted; the last arrival therefore sees every record, which it reads with sc1 loads.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ uint32_t arrived;
    uint32_t *ctr = a.counters + (uint64_t) b * nkb + kbi;
    if (threadIdx.x == 0)
        arrived = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != nsplit - 1u) return;
    const uint64_t rstride = (uint64_t) G * MOEARC_PARTIAL_FLOATS;
    constexpr int BATCH = 16;
    for (uint32_t idx = threadIdx.x; idx < KB * n_out; idx += 64u * WAVES) {
        const uint32_t k2 = idx / n_out, e = idx - k2 * n_out;
        const uint32_t kv2 = kbi * KB + k2;
        if (kv2 >= G) break;
        const uint32_t hn = e >> 6, d = e & 63u;
        const float *rec0 = a.ws + ((uint64_t) ib * G + kv2) * MOEARC_PARTIAL_FLOATS;
        float M = -INFINITY, L = 0.f, acc = 0.f;
        for (uint32_t s0 = 0; s0 < nsplit; s0 += BATCH) {
            float v[BATCH], ms[BATCH], ls[BATCH];
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const float *r = rec0 + min(s0 + (uint32_t) k, nsplit - 1u) * rstride;
                v[k] = ld_agent(r + 32u + e);
                ms[k] = ld_agent(r + hn);
                ls[k] = ld_agent(r + 16u + hn);
            }
            float mr = M;
#pragma unroll
            for (int k = 0; k < BATCH; ++k) mr = fmaxf(mr, ms[k]);  // duplicates are harmless
            const float corr = exp2_fast(M - mr);  // first batch: exp2(-inf) = 0
            L *= corr;
            acc *= corr;
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const float f = s0 + (uint32_t) k < nsplit ? exp2_fast(ms[k] - mr) : 0.f;
                L = fmaf(ls[k], f, L);
                acc = fmaf(v[k], f, acc);
            }
            M = mr;
        }
        write_output(a, b, kv2 * group + hn, d, M, L, acc);
    }
    // leave the counter at zero for the next launch (ordered before it by the kernel boundary)
    if (threadIdx.x == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split merge: for every sequence whose span was split (records are [item][kv head]), one
// MOEARC_MERGE_THREADS (256) work-group per (sequence, query head, quarter of the 64 channels), so a
// launch has four work-groups per head (grid x: head and quarter, y: sequence). Lane (sg, c) owns channel c of the quarter for the splits
// sg, sg + 16, ...; it issues every load of a round (its channel, and each split's max and
// denominator) before using any, so up to 16 * MERGE_BATCH splits cost one memory round trip.
// The 16 split groups then combine by shuffles within a wave and through LDS across the four
// waves. Runs as the next launch on the stream: the kernel boundary makes the records visible,
// with no device-scope cache maintenance inside either kernel (merging inside one launch needs a
// device-scope release -- an L2 write-back -- in every work-group, measured to cost more than
// this second launch).
#ifndef MERGE_BATCH
#define MERGE_BATCH 16
#endif

// (m, l, o) of two partial softmax sums over disjoint key sets, combined in the frame of the
// larger max; a side that saw no keys has m = -inf and drops out.
__device__ __forceinline__ void merge_partial(float &m, float &l, float &o, float m2, float l2, float o2) {
    const float M = fmaxf(m, m2);
    const float f1 = m == -INFINITY ? 0.f : exp2_fast(m - M);
    const float f2 = m2 == -INFINITY ? 0.f : exp2_fast(m2 - M);
    m = M;
    l = l * f1 + l2 * f2;
    o = o * f1 + o2 * f2;
}

extern "C" __global__ __launch_bounds__(MOEARC_MERGE_THREADS) void moearc_attn_decode_merge(const DecodeArgs a) {
    __shared__ float red[4][3][16];  // [wave][m, l, o][channel]
    const uint32_t tid = threadIdx.x, c = tid & 15u, sg = tid >> 4, wave = tid >> 6;
    // grid: x = (query head, channel quarter), y = sequence -- the sequence's item range needs no
    // load before it can be read
    const uint32_t b = blockIdx.y;
    const uint32_t ib0 = a.item_begin[b], ib1 = a.item_begin[b + 1];
    const uint32_t G = a.n_kv_heads, group = a.group;
    const uint32_t hh = blockIdx.x / MOEARC_MERGE_PARTS, part = blockIdx.x % MOEARC_MERGE_PARTS;
    const uint32_t nsplit = ib1 - ib0;
    if (nsplit <= 1u) return;  // finished by the split kernel itself
    const uint32_t kvh = hh / group, hn = hh - kvh * group;
    const uint32_t d = 16u * part + c;
    const float *rec0 = a.ws + ((uint64_t) ib0 * G + kvh) * MOEARC_PARTIAL_FLOATS;
    const uint64_t rstride = (uint64_t) G * MOEARC_PARTIAL_FLOATS;
    float m_t = -INFINITY, l_t = 0.f, o_t = 0.f;
    for (uint32_t s0 = sg; s0 < nsplit; s0 += 16u * MERGE_BATCH) {
        float v[MERGE_BATCH], ms[MERGE_BATCH], ls[MERGE_BATCH];
#pragma unroll
        for (int k = 0; k < MERGE_BATCH; ++k) {
            const uint32_t s = min(s0 + 16u * (uint32_t) k, nsplit - 1u);
            const float *r = rec0 + s * rstride;
            v[k] = r[32u + hn * 64u + d];
            ms[k] = r[hn];
            ls[k] = r[16u + hn];
        }
        float mr = m_t;
#pragma unroll
        for (int k = 0; k < MERGE_BATCH; ++k) mr = fmaxf(mr, ms[k]);  // duplicates are harmless
        const float corr = exp2_fast(m_t - mr);  // first round: exp2(-inf) = 0
        l_t *= corr;
        o_t *= corr;
#pragma unroll
        for (int k = 0; k < MERGE_BATCH; ++k) {
            const bool live = s0 + 16u * (uint32_t) k < nsplit;
            const float f = live ? exp2_fast(ms[k] - mr) : 0.f;
            l_t = fmaf(ls[k], f, l_t);
            o_t = fmaf(v[k], f, o_t);
        }
        m_t = mr;
    }
    // the four split groups of this wave (lanes c, c + 16, c + 32, c + 48)
#pragma unroll
    for (int x = 16; x <= 32; x <<= 1)
        merge_partial(m_t, l_t, o_t, __shfl_xor(m_t, x), __shfl_xor(l_t, x), __shfl_xor(o_t, x));
    if ((tid & 63u) < 16u) {
        red[wave][0][c] = m_t;
        red[wave][1][c] = l_t;
        red[wave][2][c] = o_t;
    }
    __syncthreads();
    if (tid < 16u) {
#pragma unroll
        for (int w = 1; w < 4; ++w) merge_partial(m_t, l_t, o_t, red[w][0][c], red[w][1][c], red[w][2][c]);
        write_output(a, b, hh, d, m_t, l_t, o_t);
    }
}

#define DECODE_KERNEL(KB, WPK)                                                               \
    extern "C" __global__ __launch_bounds__(64 * KB * WPK) void                             \
        moearc_attn_decode_f16d64_k##KB##w##WPK(const DecodeArgs a) {                        \
        decode_body<KB, WPK>(a);                                                            \
    }

DECODE_KERNEL(1, 4)
DECODE_KERNEL(1, 16)
DECODE_KERNEL(2, 8)
DECODE_KERNEL(4, 4)
DECODE_KERNEL(8, 2)
DECODE_KERNEL(1, 8)
DECODE_KERNEL(2, 4)
