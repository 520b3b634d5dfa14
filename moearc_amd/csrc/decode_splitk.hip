// Split-K single-query paged attention for f16 KV with head_dim 64 (the gpt-oss shape: 64 query
// heads over 8 KV heads), on gfx950 MFMA.
//
// Semantics are moearc_attn_decode's (kernels.cpp:1837-1919): for each query head,
//     out = sum_j e^(s_j - M) V_j / (e^(sink - M) + sum_j e^(s_j - M)),  s_j = scale * q.K_j,
// over the span [kv_begin, n_kv) read through the block table.
//
// Work decomposition. A work-group of KB x WPK wavefronts owns KB consecutive KV heads of one
// split (a run of split_len consecutive keys) of one sequence, and serves every query head of each
// KV head's group from a single read of each K/V row -- the KV bytes cross HBM once, not once per
// query head. The split is walked in chunks of WPK * TILES 32-key tiles; wave (kl, sub) takes KV
// head kl and the sub-th run of TILES consecutive tiles of every chunk, so the work-group reads
// KB * 128 contiguous bytes of every key row of the chunk. A wave issues every load of its chunk
// (TILES tiles, 8 x 16 bytes per lane each) before it computes any of them: at TILES = 4 that is
// 32 KiB per wave in flight, and with 8 waves per CU the whole 256 KiB share of a CU in a 32K-key
// call is requested one block-table round trip after launch. The waves merge in LDS; a sequence
// whose span fits one split is finished there (sink applied, output written); otherwise each
// work-group writes per-head partial records (max, denominator, unnormalised output) and
// moearc_attn_decode_merge, the next launch on the stream, combines them.
//
// Per 32-key tile (one wave), all operands in registers, no LDS:
//   loads   K and V rows go from HBM straight into MFMA A-operand layout: lane (g, m) loads 16
//           bytes, channels 8g..8g+7 (and 32+8g..) of key 16*blk + m.
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
//
// Kernel arguments: the fields the first loads depend on (KV and block-table bases, q, sequence
// 0's span and split, the geometry) lead the argument list as scalars, which the dispatcher
// preloads into SGPRs (the code object is built with kernarg preloading), so the block-table
// loads leave with no kernel-argument round trip before them; the rest follows as a struct read
// on demand.
#include "common.h"

// Scores live in the log2 domain, x = scale * log2(e) * q.K. Probabilities enter the f16 MFMA
// operands as p * 2^LOG2_PSCALE relative to a per-head reference max m_ref that is only moved
// when a tile's max exceeds it by more than RESCALE_SLACK (the running sums are then rescaled
// once); so p * 2^7 <= 2^(7 + 8) = 32768 stays inside f16, and p_lo (the f16 residual of p_hi)
// stays a normal f16 down to p ~ 2^-10 of the reference, with a 2^-31 floor below that.
#define LOG2_PSCALE 7.0f
#define RESCALE_SLACK 8.0f

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

// The fixed record array of the allocation-free entry point (moearc_attn_decode_batched_noalloc):
// partial records live here instead of in the context's workspace. Each loaded instance of the code
// object -- one per context, on that context's device -- holds its own array for the life of the
// module; the host takes its device address from the module (hipModuleGetGlobal, the module form of
// hipGetSymbolAddress) once, at context creation, and passes that address to the kernels like any
// workspace. External linkage so the module can name it; nothing else refers to it. Nothing in it
// needs clearing: a call's merge reads only records its own split kernel wrote.
__device__ __align__(256) float moearc_decode_scratch[MOEARC_DECODE_SCRATCH_FLOATS];

// Agent-scope relaxed atomic stores for the partial records: global_store with sc1, written
// through to the device-coherent level, so the kernel-end release has no dirty L2 lines of them
// to write back.
__device__ __forceinline__ void st_agent(float *p, float v) {
    __hip_atomic_store((uint32_t *) p, __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Final normalisation with the sink (kernels.cpp:1864-1880), in the log2 domain and the m-frame:
// out = O 2^(M-Mt) / (L 2^(M-Mt) + 2^(sink*log2e - Mt + LOG2_PSCALE)), Mt = max(M, sink*log2e).
__device__ __forceinline__ float finish(float sink2, float M, float L, float acc) {
    const float Mt = fmaxf(M, sink2);
    const float fm = exp2_fast(M - Mt);
    const float den = L * fm + exp2_fast(sink2 - Mt + LOG2_PSCALE);
    return acc * fm / den;
}

__device__ __forceinline__ void store_out(void *out, uint32_t out_f16, uint64_t o, float r) {
    if (out_f16) ((_Float16 *) out)[o] = (_Float16) r;
    else ((float *) out)[o] = r;
}

// The split kernel. Geometry words: geo0 = pt_shift | n_kv_heads << 16, geo1 = nkb | group << 16,
// nkb being the KV-head blocks (of KB heads) per work item.
template <int KB, int WPK, int TILES>
__device__ __forceinline__ void decode_body(const uint16_t *k_pages, const uint16_t *v_pages,
                                            const uint32_t *bt0, const float *q0, uint32_t kvb0,
                                            uint32_t nkv0, uint32_t slen0, uint32_t next0,
                                            uint32_t geo0, uint32_t geo1, const DecodeArgs &a) {
    constexpr int WAVES = KB * WPK;
    constexpr uint32_t CHUNK = 32u * TILES * WPK;  // keys of one chunk of the split
    // a head's 64 partial outputs per row, rows 68 floats apart: the float4 writes of a 16-lane pass
    // (16 heads, one channel quad each) then fall on 64 distinct banks (a 64-float stride put all
    // 16 heads on the same 16 banks)
    constexpr uint32_t OROW = 68;
    __shared__ float o_lds[WAVES][16 * OROW];
    __shared__ float m_lds[WAVES][16];
    __shared__ float l_lds[WAVES][16];

    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t sh = geo0 & 0xFFFFu, G = geo0 >> 16;
    const uint32_t nkb = geo1 & 0xFFFFu, group = geo1 >> 16;
    const uint32_t kbi = blockIdx.x % nkb;
    const uint32_t item = blockIdx.x / nkb;
    // Sequence 0 comes from the preloaded arguments; later sequences search the struct.
    uint32_t b = 0, ib = 0, next = next0, kvb = kvb0, nkv = nkv0, slen = slen0;
    const uint32_t *bt = bt0;
    const float *qb = q0;
    if (item >= next) {
        do ++b; while (item >= a.item_begin[b + 1]);
        ib = a.item_begin[b];
        next = a.item_begin[b + 1];
        kvb = a.kv_begin[b];
        nkv = a.n_kv[b];
        slen = a.split_len[b];
        bt = a.block_tables + (uint64_t) b * a.bt_stride;
        qb = a.q + (uint64_t) b * G * group * 64u;
    }
    const uint32_t split = item - ib;
    const uint32_t nsplit = next - ib;
    const uint32_t tb = kvb + split * slen;
    const uint32_t te = min(nkv, tb + slen);
    const uint32_t kl = wave % KB, sub = wave / KB;
    const uint32_t kvh_raw = kbi * KB + kl;
    const bool kvh_ok = kvh_raw < G;
    const uint32_t kvh = min(kvh_raw, G - 1u);
    const uint32_t g = lane >> 4, n = lane & 15u, m16 = lane & 15u;
    const bool head_ok = kvh_ok && n < group;
    const uint32_t h = kvh * group + (n < group ? n : 0u);
    const uint64_t row_elems = (uint64_t) G * 64u;
    const uint32_t pmask = (1u << sh) - 1u;

    // Block-table entries of this lane's keys in TILES tiles from key jw (j = jw + 32t + 16blk +
    // m16, clamped into the span: a tile past the span repeats its last key and computes to
    // nothing), then the physical rows once they have arrived.
    auto pages_of = [&](uint32_t jw_, uint32_t (&pid)[TILES][2]) {
#pragma unroll
        for (int t = 0; t < TILES; ++t)
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) pid[t][blk] = bt[min(jw_ + 32u * t + 16u * blk + m16, te - 1u) >> sh];
    };
    auto load_chunk = [&](uint32_t jw_, TileRegs (&r)[TILES], const uint32_t (&pid)[TILES][2]) {
#pragma unroll
        for (int t = 0; t < TILES; ++t)
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
                const uint32_t j = min(jw_ + 32u * t + 16u * blk + m16, te - 1u);
                const uint32_t row = (pid[t][blk] << sh) | (j & pmask);
                const uint64_t off = (uint64_t) row * row_elems + (uint64_t) kvh * 64u + 8u * g;
                const uint16_t *ks = k_pages + off;
                const uint16_t *vs = v_pages + off;
                r[t].k[blk][0] = *(const u32x4_t *) ks;
                r[t].k[blk][1] = *(const u32x4_t *) (ks + 32);
                r[t].v[blk][0] = *(const u32x4_t *) vs;
                r[t].v[blk][1] = *(const u32x4_t *) (vs + 32);
            }
    };

    SoftmaxState st;
    st.m = -INFINITY;
    st.l = 0.f;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) st.O[mb] = (float4_t){0.f, 0.f, 0.f, 0.f};
    uint32_t jw = tb + 32u * TILES * sub;   // this wave's first tile
    const bool active = kvh_ok && jw < te;  // uniform per wave
    if (active) {
        // ---- start-up: q and the first chunk's block-table entries leave together; the chunk's KV
        // loads leave as soon as the entries arrive, before the q arithmetic.
        float qv[16];
        const float *qrow = qb + (uint64_t) h * 64u;
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
        uint32_t pid[TILES][2];
        pages_of(jw, pid);
        TileRegs r[TILES];
        load_chunk(jw, r, pid);
        __builtin_amdgcn_sched_barrier(0);

        // Normalise each head's q by a power of two (exact) so that the hi/lo split keeps full
        // relative precision whatever q's magnitude; the inverse power folds into the score
        // multiplier.
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
            for (int i = 0; i < 8; ++i)
                sel[s][i] = (8u * g + i == 16u * s + n) ? (_Float16) 1.0f : (_Float16) 0.0f;

        // ---- key loop: every load of a chunk is issued before any of its tiles is computed, and
        // the next chunk's block-table entries leave before the computing starts. (The compiler
        // drains the next chunk's KV loads at the back edge; they were all issued together, so the
        // first tile would wait for nearly as long anyway.)
        for (;;) {
            const uint32_t jn = jw + CHUNK;
            const bool more = jn < te;  // uniform
            pages_of(more ? jn : jw, pid);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TILES; ++t) process_tile(st, r[t], qhi, qlo, sel, c, jw + 32u * t, te, g);
            if (!more) break;
            jw = jn;
            load_chunk(jw, r, pid);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- merge the WPK waves of each KV head in LDS ---------------------------------------------
    float l_run = st.l;
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (head_ok) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
            *(float4_t *) (&o_lds[wave][n * OROW + 16u * mb + 4u * g]) = st.O[mb];
    }
    if (g == 0) {
        m_lds[wave][n] = head_ok && active ? st.m : -INFINITY;
        l_lds[wave][n] = head_ok && active ? l_run : 0.f;
    }
    __syncthreads();

    // Threads take (KV head of the block, output element) pairs.
    const uint32_t n_out = group * 64u;
    const bool single = nsplit == 1u;
    const uint32_t H = G * group;
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
            const float mw = m_lds[ww][hn];
            const float f = mw == -INFINITY ? 0.f : exp2_fast(mw - M);  // a wave without keys drops out
            L += l_lds[ww][hn] * f;
            acc += o_lds[ww][hn * OROW + d] * f;
        }
        const uint32_t hh = kv2 * group + hn;
        if (single) {
            const float sink2 = a.sinks ? a.sinks[hh] * MOEARC_LOG2E : -INFINITY;
            store_out(a.out, a.out_f16, ((uint64_t) b * H + hh) * 64u + d, finish(sink2, M, L, acc));
        } else {
            // records, head-major: [head][work item], so a head's splits are contiguous
            const uint64_t r_i = (uint64_t) hh * a.n_items + item;
            st_agent(a.rec_o + r_i * 64u + d, acc);
            if (d == 0) {
                st_agent(a.rec_ml + 2u * r_i, M);
                st_agent(a.rec_ml + 2u * r_i + 1u, L);
            }
        }
    }
}

#define DECODE_KERNEL(KB, WPK, TILES)                                                          \
    extern "C" __global__ __launch_bounds__(64 * KB * WPK) void                               \
        moearc_attn_decode_f16d64_k##KB##w##WPK##t##TILES(                                     \
            const uint16_t *k_pages, const uint16_t *v_pages, const uint32_t *bt0,             \
            const float *q0, uint32_t kvb0, uint32_t nkv0, uint32_t slen0, uint32_t next0,     \
            uint32_t geo0, uint32_t geo1, const DecodeArgs a) {                                \
        decode_body<KB, WPK, TILES>(k_pages, v_pages, bt0, q0, kvb0, nkv0, slen0, next0,       \
                                    geo0, geo1, a);                                            \
    }

DECODE_KERNEL(4, 2, 4)  // long spans: 8 waves, 256-key chunks, 32 KiB per wave in flight
DECODE_KERNEL(1, 4, 1)  // short spans: 4 waves, 128-key chunks, many work-groups

// (m, l, o) of two partial softmax sums over disjoint key sets, combined in the frame of the
// larger max; a side that saw no keys has m = -inf and drops out.
__device__ __forceinline__ void merge_partial4(float &m, float &l, float4_t &o, float m2, float l2,
                                               float4_t o2) {
    const float M = fmaxf(m, m2);
    const float f1 = m == -INFINITY ? 0.f : exp2_fast(m - M);
    const float f2 = m2 == -INFINITY ? 0.f : exp2_fast(m2 - M);
    m = M;
    l = l * f1 + l2 * f2;
    o = o * f1 + o2 * f2;
}

// Split merge. PARTS 256-thread work-groups per (query head, sequence), each owning 64 / PARTS
// output channels (one: measured as fast as four at config 2's 128 splits, and a quarter of the
// work-groups): lane (split group sg, channel quad c4) owns channels 4c4..4c4+3 of the part for
// the splits sg, sg + NSG, ...; it issues every load of a round (a 16-byte piece of each of
// MERGE_BATCH records and their (max, denominator) pairs) before using any, so up to
// NSG * MERGE_BATCH splits cost one memory round trip, and a head's records are contiguous. The
// split groups then combine by shuffles within a wave and through LDS across the four waves.
// Arguments: record bases, output, sinks and sequence 0's item count are preloaded scalars; the
// struct carries the other sequences' item ranges.
#define MERGE_BATCH 8

template <int PARTS>
__device__ __forceinline__ void merge_body(const float *rec_o, const float *rec_ml, void *out,
                                           const float *sinks, uint32_t n_items, uint32_t next0,
                                           uint32_t n_heads, uint32_t out_f16, const MergeArgs &ma) {
    constexpr uint32_t QUADS = 16 / PARTS, NSG = MOEARC_MERGE_THREADS / QUADS;
    __shared__ float red[4][6][QUADS];  // [wave][m, l, o0..o3][channel quad]
    const uint32_t tid = threadIdx.x, c4 = tid % QUADS, sg = tid / QUADS, wave = tid >> 6;
    const uint32_t b = blockIdx.y, h = blockIdx.x / PARTS, part = blockIdx.x % PARTS;
    uint32_t ib0 = 0, ib1 = next0;
    if (b > 0) {
        ib0 = ma.item_begin[b];
        ib1 = ma.item_begin[b + 1];
    }
    const uint32_t nsplit = ib1 - ib0;
    if (nsplit <= 1u) return;  // finished by the split kernel itself
    // the sink, requested with the records and first used at the end (without sinks the load reads
    // a record word, ignored)
    const float sink_raw = *(sinks ? sinks + h : rec_ml);
    const uint32_t ch = 16u * part + 4u * c4;
    const uint64_t base = (uint64_t) h * n_items + ib0;
    float m_t = -INFINITY, l_t = 0.f;
    float4_t o_t = (float4_t){0.f, 0.f, 0.f, 0.f};
    for (uint32_t s0 = sg; s0 < nsplit; s0 += NSG * MERGE_BATCH) {
        float4_t v[MERGE_BATCH];
        float2_t ml[MERGE_BATCH];
#pragma unroll
        for (int k = 0; k < MERGE_BATCH; ++k) {
            const uint64_t s = base + min(s0 + NSG * (uint32_t) k, nsplit - 1u);
            v[k] = *(const float4_t *) (rec_o + s * 64u + ch);
            ml[k] = *(const float2_t *) (rec_ml + 2u * s);
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the round leaves before any is used
        float mr = m_t;
#pragma unroll
        for (int k = 0; k < MERGE_BATCH; ++k) mr = fmaxf(mr, ml[k][0]);  // duplicates are harmless
        const float corr = m_t == -INFINITY ? 0.f : exp2_fast(m_t - mr);
        l_t *= corr;
        o_t *= corr;
#pragma unroll
        for (int k = 0; k < MERGE_BATCH; ++k) {
            const bool live = s0 + NSG * (uint32_t) k < nsplit;
            const float f = live ? exp2_fast(ml[k][0] - mr) : 0.f;
            l_t = fmaf(ml[k][1], f, l_t);
            o_t += v[k] * f;
        }
        m_t = mr;
    }
    // the split groups of this wave (lanes equal modulo QUADS)
#pragma unroll
    for (uint32_t x = QUADS; x < 64u; x <<= 1) {
        float4_t o2;
#pragma unroll
        for (int i = 0; i < 4; ++i) o2[i] = __shfl_xor(o_t[i], x);
        merge_partial4(m_t, l_t, o_t, __shfl_xor(m_t, x), __shfl_xor(l_t, x), o2);
    }
    if ((tid & 63u) < QUADS) {
        red[wave][0][c4] = m_t;
        red[wave][1][c4] = l_t;
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][2 + i][c4] = o_t[i];
    }
    __syncthreads();
    if (tid < QUADS) {
#pragma unroll
        for (int w = 1; w < 4; ++w)
            merge_partial4(m_t, l_t, o_t, red[w][0][c4], red[w][1][c4],
                           (float4_t){red[w][2][c4], red[w][3][c4], red[w][4][c4], red[w][5][c4]});
        const float sink2 = sinks ? sink_raw * MOEARC_LOG2E : -INFINITY;
        const uint64_t o = ((uint64_t) b * n_heads + h) * 64u + ch;
        float r4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) r4[i] = finish(sink2, m_t, l_t, o_t[i]);
        if (out_f16) {
            half2_t lo = {(_Float16) r4[0], (_Float16) r4[1]}, hi = {(_Float16) r4[2], (_Float16) r4[3]};
            *(half2_t *) ((_Float16 *) out + o) = lo;
            *(half2_t *) ((_Float16 *) out + o + 2) = hi;
        } else {
            *(float4_t *) ((float *) out + o) = (float4_t){r4[0], r4[1], r4[2], r4[3]};
        }
    }
}

#define MERGE_KERNEL(PARTS)                                                                    \
    extern "C" __global__ __launch_bounds__(MOEARC_MERGE_THREADS) void                        \
        moearc_attn_decode_merge_p##PARTS(const float *rec_o, const float *rec_ml, void *out,  \
                                          const float *sinks, uint32_t n_items, uint32_t next0, \
                                          uint32_t n_heads, uint32_t out_f16, const MergeArgs ma) { \
        merge_body<PARTS>(rec_o, rec_ml, out, sinks, n_items, next0, n_heads, out_f16, ma);    \
    }

MERGE_KERNEL(1)
