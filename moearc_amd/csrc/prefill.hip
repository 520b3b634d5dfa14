// Chunked prefill over a paged f16 KV cache, head_dim 64, on gfx950 MFMA.
//
// Semantics are the reference engine's prefill -- one decode per prompt token
// (moe.rs:1856-1862, session.rs:378-381): query row i sits at absolute position p = pos0 + i, its own
// K/V already in the cache, and attends keys [b(p), p] with b(p) = max(0, p + 1 - n_swa) on a
// windowed layer (moe.rs:2020-2027) and 0 otherwise; the per-head sink enters the denominator as in
// decode (kernels.cpp:1864-1880).
//
// Work decomposition. A work-group owns one KV head and 128 query rows, a row being one
// (token, head) pair of that KV head's group -- GQA packing, so every K/V tile staged in LDS serves
// all the group's heads. Four waves take 32 rows each. Keys stream through LDS in 64-key tiles,
// double-buffered: the next tile's global loads are in flight while the current one is computed.
//
// LDS layouts (per buffer, 16 KiB):
//   K  [64 keys][64 ch] f16, 16-byte chunks XOR-swizzled by (key & 7): the QK^T A-operand read --
//      lane (g, m) takes channels 8g..8g+7 (+32) of key m -- is one conflict-free ds_read_b128.
//   V^T [64 ch][64 keys] f16, 8-byte units XOR-swizzled by (ch & 15): the P.V A-operand -- lane
//      (g, m) takes keys 4g..4g+3 and 16+4g..16+4g+3 of channel m -- is two ds_read_b64. The
//      transpose happens on the LDS write: each thread packs two keys' values of one channel into
//      a dword (v_perm) and stores it.
// Per 32-key chunk, a wave computes S^T[32 keys x 32 rows] = K . Q^T (8 MFMAs, f16 Q is exact),
// the online softmax in the log2 domain with a lazily moved reference max, and
// O^T[64 ch x 32 rows] += V^T . P^T (8 MFMAs) with P as one f16 operand, f32 accumulation: the
// weights carry f16's 11 bits, an output error of at most 2^-12 max|V| (measured ~2.5e-4 on N(0,1)
// data). The _precise_ variants split p = p_hi + p_lo into two f16 operands (16 MFMAs), keeping
// ~22 bits like the decode kernel. Causal/window masks are applied only in chunks that cross a
// row's span boundary.
#include "common.h"

#define PF_LOG2_PSCALE 7.0f
#define PF_RESCALE_SLACK 8.0f
#define PF_M_INIT -1.0e30f  // finite "no key yet": keeps exp2(m_old - m_new) defined for rows
                            // whose keys all lie in later chunks
#define PF_PT_CAP 2048      // block-table entries staged in LDS per work-group
#define PF_KT 64            // keys per LDS tile

__device__ __forceinline__ float4_t pf_mfma(const half8_t a, const half8_t b, const float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float pf_max16_32(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

// Byte offset of K element chunk c (8 channels) of key k within a K tile.
__device__ __forceinline__ uint32_t k_off(uint32_t k, uint32_t c) {
    return k * 128u + ((c ^ (k & 7u)) << 4);
}

// Byte offset of the dword holding keys (k, k+1) (k even) of channel d within a V^T tile.
__device__ __forceinline__ uint32_t vt_off(uint32_t d, uint32_t k) {
    return d * 128u + ((((k >> 2) ^ (d & 15u))) << 3) + ((k & 3u) << 1);
}

template <int GROUP, bool SPLIT_P>
__device__ __forceinline__ void prefill_body(const PrefillArgs &a) {
    constexpr uint32_t ROWS = MOEARC_PREFILL_ROWS;  // 128 rows per work-group
    constexpr uint32_t TOK = ROWS / GROUP;          // query tokens per work-group
    __shared__ __attribute__((aligned(16))) uint8_t kv_lds[2][2][PF_KT * 128];  // [buf][K, V^T]
    __shared__ uint32_t pt_lds[PF_PT_CAP];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = a.n_kv_heads;
    const uint32_t kvh = blockIdx.x % G;
    const uint32_t qt = blockIdx.x / G;
    const uint32_t q0 = qt * TOK;                   // first query token of the work-group
    const uint32_t q_end = min(q0 + TOK, a.n_q);
    const uint32_t g = lane >> 4, n = lane & 15u;
    const uint32_t sh = a.pt_shift;

    // key span of the whole work-group
    const uint32_t p_first = a.pos0 + q0, p_last = a.pos0 + q_end - 1u;
    const uint32_t k_lo = a.n_swa ? (p_first + 1u > a.n_swa ? p_first + 1u - a.n_swa : 0u) : 0u;
    const uint32_t kt_first = k_lo / PF_KT, kt_last = p_last / PF_KT;
    const uint32_t page0 = (kt_first * PF_KT) >> sh;
    const uint32_t npages = (p_last >> sh) - page0 + 1u;  // host guarantees <= PF_PT_CAP
    for (uint32_t i = tid; i < npages; i += 256u) pt_lds[i] = a.block_table[page0 + i];

    // ---- rows of this wave: local row r (0..31) -> (token, head) --------------------------------
    // Q^T operand: lane (g, n) of row block rb holds row 16*rb + n, channels 32*hf + 8g .. +7
    half8_t qop[2][2];
    uint32_t row_pos[2];   // absolute position of the row lane n holds in each row block
    bool row_ok[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const uint32_t r = wave * 32u + 16u * rb + n;  // work-group row
        const uint32_t tok = q0 + r / GROUP, hd = kvh * GROUP + r % GROUP;
        row_ok[rb] = tok < q_end;
        row_pos[rb] = a.pos0 + min(tok, q_end - 1u);
        const uint16_t *src = a.q + ((uint64_t) min(tok, a.n_q - 1u) * a.n_heads + hd) * 64u + 8u * g;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            u32x4_t v = *(const u32x4_t *) (src + 32 * hf);
            if (!row_ok[rb]) v = (u32x4_t){0u, 0u, 0u, 0u};
            qop[rb][hf] = __builtin_bit_cast(half8_t, v);
        }
    }
    // the wave's position range, for deciding which chunks need masks
    const uint32_t w_tok0 = q0 + (wave * 32u) / GROUP;
    const uint32_t w_tok1 = min(q0 + (wave * 32u + 31u) / GROUP, q_end - 1u);
    const uint32_t w_pmin = a.pos0 + min(w_tok0, q_end - 1u), w_pmax = a.pos0 + w_tok1;
    const uint32_t w_bmin = a.n_swa ? (w_pmin + 1u > a.n_swa ? w_pmin + 1u - a.n_swa : 0u) : 0u;
    const uint32_t w_bmax = a.n_swa ? (w_pmax + 1u > a.n_swa ? w_pmax + 1u - a.n_swa : 0u) : 0u;

    const float c = a.scale_log2e;
    float m_run[2] = {PF_M_INIT, PF_M_INIT};
    float l_run[2] = {0.f, 0.f};
    float4_t O[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) O[mb][rb] = (float4_t){0.f, 0.f, 0.f, 0.f};

    __syncthreads();  // page table staged

    // ---- global -> registers for one tile: thread t takes K chunk (key t/8 and t/8+32, ch t%8) --
    // and V rows (keys 2*(t/8), 2*(t/8)+1, ch t%8)
    const uint32_t ld_k = tid >> 3, ld_c = tid & 7u;
    const uint64_t row_elems = (uint64_t) G * 64u;
    auto key_addr = [&](uint32_t j) -> uint64_t {
        const uint32_t jc = min(j, p_last);
        const uint32_t row = (pt_lds[(jc >> sh) - page0] << sh) | (jc & ((1u << sh) - 1u));
        return (uint64_t) row * row_elems + (uint64_t) kvh * 64u + 8u * ld_c;
    };
    u32x4_t gk[2], gv[2];
    auto gload = [&](uint32_t kt) {
        const uint32_t j0 = kt * PF_KT;
        gk[0] = *(const u32x4_t *) (a.k_pages + key_addr(j0 + ld_k));
        gk[1] = *(const u32x4_t *) (a.k_pages + key_addr(j0 + ld_k + 32u));
        gv[0] = *(const u32x4_t *) (a.v_pages + key_addr(j0 + 2u * ld_k));
        gv[1] = *(const u32x4_t *) (a.v_pages + key_addr(j0 + 2u * ld_k + 1u));
    };
    auto lds_store = [&](int buf) {
        uint8_t *kb = kv_lds[buf][0], *vb = kv_lds[buf][1];
        *(u32x4_t *) (kb + k_off(ld_k, ld_c)) = gk[0];
        *(u32x4_t *) (kb + k_off(ld_k + 32u, ld_c)) = gk[1];
        // channel 8*ld_c + e of keys (2*ld_k, 2*ld_k + 1) -> one dword of V^T
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = __builtin_amdgcn_perm(gv[1][e], gv[0][e], 0x05040100u);  // ch 2e
            const uint32_t hi = __builtin_amdgcn_perm(gv[1][e], gv[0][e], 0x07060302u);  // ch 2e+1
            *(uint32_t *) (vb + vt_off(8u * ld_c + 2u * e, 2u * ld_k)) = lo;
            *(uint32_t *) (vb + vt_off(8u * ld_c + 2u * e + 1u, 2u * ld_k)) = hi;
        }
    };

    gload(kt_first);
    lds_store(0);
    __syncthreads();
    int buf = 0;
    for (uint32_t kt = kt_first; kt <= kt_last; ++kt) {
        const bool more = kt < kt_last;
        if (more) gload(kt + 1u);  // uniform branch: the last tile has nothing to prefetch
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
        const uint8_t *kb = kv_lds[buf][0], *vb = kv_lds[buf][1];
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {  // 32-key chunks
            const uint32_t j0 = kt * PF_KT + 32u * kc;
            if (j0 > w_pmax || j0 + 31u < w_bmin) continue;  // no row of this wave sees the chunk
            // QK^T: S[kb2][rb] lane (g, n) reg i = key j0 + 16*kb2 + 4g + i, row 16*rb + n
            float4_t S[2][2];
#pragma unroll
            for (int kb2 = 0; kb2 < 2; ++kb2) {
                const uint32_t key = 32u * kc + 16u * kb2 + n;  // A-operand row = lane n
                const half8_t k0 = __builtin_bit_cast(half8_t, *(const u32x4_t *) (kb + k_off(key, g)));
                const half8_t k1 = __builtin_bit_cast(half8_t, *(const u32x4_t *) (kb + k_off(key, 4u + g)));
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    float4_t s = (float4_t){0.f, 0.f, 0.f, 0.f};
                    s = pf_mfma(k0, qop[rb][0], s);
                    s = pf_mfma(k1, qop[rb][1], s);
                    S[kb2][rb] = s;
                }
            }
            // masks, only where the chunk crosses some row's span boundary (uniform branch)
            if (j0 + 31u > w_pmin || (a.n_swa && j0 < w_bmax)) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    const uint32_t p = row_pos[rb];
                    const uint32_t bp = a.n_swa ? (p + 1u > a.n_swa ? p + 1u - a.n_swa : 0u) : 0u;
#pragma unroll
                    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t j = j0 + 16u * kb2 + 4u * g + i;
                            if (j > p || j < bp) S[kb2][rb][i] = -INFINITY;
                        }
                }
            }
            // online softmax per row block; P^T operand item i = key 16*(i/4) + 4g + i%4
            half8_t phi[2], plo[2];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                float tmax = fmaxf(fmaxf(fmaxf(S[0][rb][0], S[0][rb][1]), fmaxf(S[0][rb][2], S[0][rb][3])),
                                   fmaxf(fmaxf(S[1][rb][0], S[1][rb][1]), fmaxf(S[1][rb][2], S[1][rb][3])));
                tmax = pf_max16_32(tmax) * c;
                if (__builtin_amdgcn_ballot_w64(tmax > m_run[rb] + PF_RESCALE_SLACK) != 0) {
                    const float m_new = fmaxf(m_run[rb], tmax);
                    const float corr = __builtin_amdgcn_exp2f(m_run[rb] - m_new);
                    m_run[rb] = m_new;
                    l_run[rb] *= corr;
#pragma unroll
                    for (int mb = 0; mb < 4; ++mb) O[mb][rb] *= corr;
                }
                const float bias = PF_LOG2_PSCALE - m_run[rb];
                float psum = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float ps = __builtin_amdgcn_exp2f(fmaf(S[i >> 2][rb][i & 3], c, bias));
                    psum += ps;
                    const _Float16 hi = (_Float16) ps;
                    phi[rb][i] = hi;
                    if constexpr (SPLIT_P) plo[rb][i] = (_Float16) (ps - (float) hi);
                }
                l_run[rb] += psum;
            }
            // P.V: V^T operand for channel block mb: lane (g, m) = channel 16*mb + m,
            // keys 32*kc + 4g .. +3 and 32*kc + 16 + 4g .. +3
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const uint32_t d = 16u * mb + n;
                const uint32_t base = d * 128u;
                const uint32_t u0 = 8u * kc + g, u1 = 8u * kc + 4u + g;  // 8-byte units (4 keys)
                const uint64_t lo4 = *(const uint64_t *) (vb + base + ((u0 ^ (d & 15u)) << 3));
                const uint64_t hi4 = *(const uint64_t *) (vb + base + ((u1 ^ (d & 15u)) << 3));
                const u32x4_t vv = (u32x4_t){(uint32_t) lo4, (uint32_t) (lo4 >> 32), (uint32_t) hi4,
                                             (uint32_t) (hi4 >> 32)};
                const half8_t va = __builtin_bit_cast(half8_t, vv);
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    O[mb][rb] = pf_mfma(va, phi[rb], O[mb][rb]);
                    if constexpr (SPLIT_P) O[mb][rb] = pf_mfma(va, plo[rb], O[mb][rb]);
                }
            }
        }
        __syncthreads();  // every wave is done reading this buffer and (as of the loop head) the other
        if (more) {
            lds_store(buf ^ 1);
            __syncthreads();
            buf ^= 1;
        }
    }

    // ---- finalise: denominators over the 4 lanes of a row, the sink, the store -----------------
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        float L = l_run[rb];
        L += __shfl_xor(L, 16);
        L += __shfl_xor(L, 32);
        const uint32_t r = wave * 32u + 16u * rb + n;
        const uint32_t tok = q0 + r / GROUP, hd = kvh * GROUP + r % GROUP;
        const float sink2 = a.sinks ? a.sinks[hd] * MOEARC_LOG2E : -INFINITY;
        const float M = m_run[rb];
        const float Mt = fmaxf(M, sink2);
        const float fm = __builtin_amdgcn_exp2f(M - Mt);
        const float inv = fm / (L * fm + __builtin_amdgcn_exp2f(sink2 - Mt + PF_LOG2_PSCALE));
        if (tok < q_end) {
            const uint64_t o = ((uint64_t) tok * a.n_heads + hd) * 64u;
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const float4_t v = O[mb][rb] * inv;
                const uint32_t d = 16u * mb + 4u * g;
                if (a.out_f16) {
                    half2_t h0 = {(_Float16) v[0], (_Float16) v[1]};
                    half2_t h1 = {(_Float16) v[2], (_Float16) v[3]};
                    uint2 w = {__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
                    *(uint2 *) ((_Float16 *) a.out + o + d) = w;
                } else {
                    *(float4_t *) ((float *) a.out + o + d) = v;
                }
            }
        }
    }
}

#define PREFILL_KERNEL(GRP)                                                                      \
    extern "C" __global__ __launch_bounds__(MOEARC_PREFILL_THREADS) void moearc_attn_prefill_g##GRP( \
        const PrefillArgs a) {                                                                   \
        prefill_body<GRP, false>(a);                                                             \
    }                                                                                            \
    extern "C" __global__ __launch_bounds__(MOEARC_PREFILL_THREADS) void                        \
        moearc_attn_prefill_precise_g##GRP(const PrefillArgs a) {                                \
        prefill_body<GRP, true>(a);                                                              \
    }

PREFILL_KERNEL(1)
PREFILL_KERNEL(2)
PREFILL_KERNEL(4)
PREFILL_KERNEL(8)
