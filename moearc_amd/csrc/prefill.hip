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
// all the group's heads. Four waves take 32 rows each. Query tiles are dispatched latest first:
// under the causal mask the latest tokens have the most keys, and the short tiles fill in behind.
//
// Keys stream through LDS in 64-key tiles, two buffers (each its own LDS object, the loop unrolled
// by two, so the compiler can tell a read of one buffer from the copy in flight into the other):
// at the top of tile kt every wave waits for its copies of tile kt and meets the others at a
// barrier, issues the copies of tile kt + 1 into the other buffer, then computes tile kt.
// The copies are global_load_lds_dwordx4 (16 bytes per lane, placed at base + 16 * lane), so tiles
// go from the cache to LDS without passing through registers; the block-table entries a lane needs
// for a tile are loaded one tile ahead.
//
// LDS layout of a buffer: K and V each [64 keys][64 ch] f16, 128-byte rows whose 16-byte chunks are
// XOR-swizzled by (key & 7): chunk c of key k at k * 128 + ((c ^ (k & 7)) << 4).
//   QK^T A-operand (K): lane (g, m) takes channels 8g..8g+7 (and +32) of key m -- one
//      ds_read_b128, conflict-free.
//   P.V A-operand (V^T): lane (g, m) needs channel m of keys {4g..4g+3} and {16+4g..16+4g+3}, the
//      MFMA k-slot order of the P operand. ds_read_b64_tr_b16 transposes within each 16-lane group
//      (lane r receives element r & 3 of the 8 bytes addressed by lanes 4j + (r >> 2), j = 0..3),
//      so lane s of group g addresses key 4g + (s >> 2) (+16), channels 4(s & 3)..+3 of the block:
//      two conflict-free reads per operand.
// Per 32-key chunk, a wave computes S^T[32 keys x 32 rows] = K . Q^T (8 MFMAs, f16 Q is exact),
// the softmax weights p = 2^(s*c + 7 - m) in the log2 domain against a lazily moved per-row
// reference m, and O^T[64 ch x 32 rows] += V^T . P^T (8 MFMAs) with P as one f16 operand, f32
// accumulation: the weights carry f16's 11 bits, an output error of at most 2^-12 max|V|
// (measured ~2.5e-4 on N(0,1) data). The row sums come from the same f16 P through two more
// MFMAs against an all-ones operand. The _precise_ variants split p = p_hi + p_lo into two f16
// operands, keeping ~22 bits like the decode kernel.
//
// The reference m moves only when some score of the row exceeds it by more than 8 (log2 units),
// which each lane detects from its own 8 scores; the cross-lane row maximum and the rescale of
// O and the sums run only then (in practice at a row's first chunk). So p <= 2^15 fits f16.
// Causal/window masks are applied only in chunks that cross a row's span boundary.
#include "common.h"

#define PF_LOG2_PSCALE 7.0f
#define PF_RESCALE_SLACK 8.0f
#define PF_M_INIT -1.0e30f  // finite "no key yet": keeps exp2(m_old - m_new) defined for rows
                            // whose keys all lie in later chunks
#define PF_KT 64            // keys per LDS tile

__device__ __forceinline__ float4_t pf_mfma(const half8_t a, const half8_t b, const float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float pf_max16_32(float x) {
    x = fmaxf(x, __shfl_xor(x, 16));
    x = fmaxf(x, __shfl_xor(x, 32));
    return x;
}

__device__ __forceinline__ float pf_max8(const float4_t a, const float4_t b) {
    return fmaxf(fmaxf(fmaxf(a[0], a[1]), fmaxf(a[2], a[3])), fmaxf(fmaxf(b[0], b[1]), fmaxf(b[2], b[3])));
}

// Byte offset of 16-byte chunk c (8 channels) of key k within a K or V tile.
__device__ __forceinline__ uint32_t kv_off(uint32_t k, uint32_t c) {
    return k * 128u + ((c ^ (k & 7u)) << 4);
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void pf_static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        pf_static_for<B + 1, E>(f);
    }
}

// LDS reads of the tiles are issued through asm, each group together with its wait: the tiles
// are filled by LDS DMA, and the compiler, which cannot tell the buffer being read from the one
// being filled, would otherwise wait for the copy in flight before every read. Offsets are
// immediates (per-lane base address + buffer/chunk offset).
template <int O0, int O1>
__device__ __forceinline__ void pf_read_k(u32x4_t (&r)[4], uint32_t a0, uint32_t a1) {
    asm volatile(
        "ds_read_b128 %0, %4 offset:%6\n\t"
        "ds_read_b128 %1, %5 offset:%6\n\t"
        "ds_read_b128 %2, %4 offset:%7\n\t"
        "ds_read_b128 %3, %5 offset:%7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(a0), "v"(a1), "i"(O0), "i"(O1)
        : "memory");
}

// Transposing reads (ds_read_b64_tr_b16) of two V^T operands: bases a0, a1, keys +0 and +16.
template <int O0, int O1>
__device__ __forceinline__ void pf_read_vt(u32x2_t (&r)[4], uint32_t a0, uint32_t a1) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %4 offset:%6\n\t"
        "ds_read_b64_tr_b16 %1, %4 offset:%7\n\t"
        "ds_read_b64_tr_b16 %2, %5 offset:%6\n\t"
        "ds_read_b64_tr_b16 %3, %5 offset:%7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(a0), "v"(a1), "i"(O0), "i"(O1)
        : "memory");
}

template <int GROUP, bool SPLIT_P>
__device__ __forceinline__ void prefill_body(const PrefillArgs &a) {
    constexpr uint32_t ROWS = MOEARC_PREFILL_ROWS;  // 128 rows per work-group
    constexpr uint32_t TOK = ROWS / GROUP;          // query tokens per work-group
    constexpr uint32_t TILE_BYTES = PF_KT * 128u;   // one K or V tile
    constexpr uint32_t BUF_BYTES = 2u * TILE_BYTES;  // K tile, V tile
    __shared__ __attribute__((aligned(1024))) uint8_t tiles[2 * BUF_BYTES];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = a.n_kv_heads;
    const uint32_t kvh = blockIdx.x % G;
    const uint32_t qt = a.n_qtiles - 1u - blockIdx.x / G;
    const uint32_t q0 = qt * TOK;                   // first query token of the work-group
    const uint32_t q_end = min(q0 + TOK, a.n_q);
    const uint32_t g = lane >> 4, n = lane & 15u;
    const uint32_t sh = a.pt_shift, pmask = (1u << sh) - 1u;

    // key span of the whole work-group
    const uint32_t p_first = a.pos0 + q0, p_last = a.pos0 + q_end - 1u;
    const uint32_t k_lo = a.n_swa ? (p_first + 1u > a.n_swa ? p_first + 1u - a.n_swa : 0u) : 0u;
    const uint32_t kt_first = k_lo / PF_KT, kt_last = p_last / PF_KT;

    // ---- rows of this wave: local row r (0..31) -> (token, head) --------------------------------
    // Q^T operand: lane (g, n) of row block rb holds row 16*rb + n, channels 32*hf + 8g .. +7
    half8_t qop[2][2];
    uint32_t row_pos[2];   // absolute position of the row lane n holds in each row block
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const uint32_t r = wave * 32u + 16u * rb + n;  // work-group row
        const uint32_t tok = q0 + r / GROUP, hd = kvh * GROUP + r % GROUP;
        const bool ok = tok < q_end;
        row_pos[rb] = a.pos0 + min(tok, q_end - 1u);
        const uint16_t *src = a.q + ((uint64_t) min(tok, a.n_q - 1u) * a.n_heads + hd) * 64u + 8u * g;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            u32x4_t v = *(const u32x4_t *) (src + 32 * hf);
            if (!ok) v = (u32x4_t){0u, 0u, 0u, 0u};
            qop[rb][hf] = __builtin_bit_cast(half8_t, v);
        }
    }
    // the wave's position range, for deciding which chunks need masks
    const uint32_t w_tok0 = q0 + (wave * 32u) / GROUP;
    const uint32_t w_tok1 = min(q0 + (wave * 32u + 31u) / GROUP, q_end - 1u);
    const uint32_t w_pmin = a.pos0 + min(w_tok0, q_end - 1u), w_pmax = a.pos0 + w_tok1;
    const uint32_t w_bmin = a.n_swa ? (w_pmin + 1u > a.n_swa ? w_pmin + 1u - a.n_swa : 0u) : 0u;
    const uint32_t w_bmax = a.n_swa ? (w_pmax + 1u > a.n_swa ? w_pmax + 1u - a.n_swa : 0u) : 0u;

    // s*c with c < 0 equals (-s)*(-c): negate the f16 Q operand (exact) so that c > 0 and the
    // row maximum of s*c is c times the maximum of s
    float c = a.scale_log2e;
    if (c < 0.f) {
        c = -c;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) qop[rb][hf] = -qop[rb][hf];
    }
    float m_run[2] = {PF_M_INIT, PF_M_INIT};
    float4_t O[4][2], Lsum[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        Lsum[rb] = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) O[mb][rb] = (float4_t){0.f, 0.f, 0.f, 0.f};
    }
    const half8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};

    // ---- per-lane LDS base addresses (buffer 0, chunk 0, tile offset excluded) ----------------
    // K operand: key n, chunks g and g + 4. V^T operand of channel block mb: key 4g + (n >> 2),
    // chunk 2mb + ((n >> 1) & 1), 8-byte half n & 1. Chunk/buffer offsets keep the swizzle (key & 7).
    const uint32_t lds0 = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) uint8_t *) tiles;
    const uint32_t k_base0 = lds0 + kv_off(n, g), k_base1 = lds0 + kv_off(n, g + 4u);
    const uint32_t vkey = 4u * g + (n >> 2);
    uint32_t v_base[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
        v_base[mb] = lds0 + kv_off(vkey, 2u * mb + ((n >> 1) & 1u)) + ((n & 1u) << 3);

    // ---- tile copies: lane L of wave w fills LDS chunk slot L of keys 16w + 8i + (L >> 3) -------
    // (i = 0, 1) of the K and the V tile; that slot holds chunk (L & 7) ^ (L >> 3) of the key.
    // Keys past p_last (no row sees them) are clamped to p_last so every copy reads a valid row.
    const uint32_t ld_key = 16u * wave + (lane >> 3);
    const uint32_t ld_chunk = (lane & 7u) ^ (lane >> 3);
    const uint64_t row_bytes = (uint64_t) G * 128u;
    const uint8_t *k_src = (const uint8_t *) a.k_pages + kvh * 128u + ld_chunk * 16u;
    const uint8_t *v_src = (const uint8_t *) a.v_pages + kvh * 128u + ld_chunk * 16u;
    uint32_t pid[2];  // block-table entries of this lane's two keys of the next tile
    auto load_pids = [&](uint32_t kt) {
#pragma unroll
        for (int i = 0; i < 2; ++i) pid[i] = a.block_table[min(kt * PF_KT + ld_key + 8u * i, p_last) >> sh];
    };
    auto copy_tile = [&](uint32_t kt, int buf) {
        uint8_t *dst = tiles + buf * BUF_BYTES;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t j = min(kt * PF_KT + ld_key + 8u * i, p_last);
            const uint64_t off = (uint64_t) ((pid[i] << sh) | (j & pmask)) * row_bytes;
            uint8_t *d = dst + (16u * wave + 8u * i) * 128u;
            __builtin_amdgcn_global_load_lds(k_src + off, d, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(v_src + off, d + TILE_BYTES, 16, 0, 0);
        }
    };

    // ---- one tile: 2 chunks of 32 keys ----------------------------------------------------------
    auto compute_tile = [&](uint32_t kt, auto buf_c) {
        constexpr int BOFF = decltype(buf_c)::value * (int) BUF_BYTES;
        pf_static_for<0, 2>([&](auto kc_c) {  // 32-key chunks
            constexpr int kc = decltype(kc_c)::value;
            const uint32_t j0 = kt * PF_KT + 32u * kc;
            if (j0 > w_pmax || j0 + 31u < w_bmin) return;  // no row of this wave sees the chunk
            // QK^T: S[kb2][rb] lane (g, n) reg i = key j0 + 16*kb2 + 4g + i, row 16*rb + n
            u32x4_t kr[4];  // [kb2 * 2 + channel half]
            pf_read_k<BOFF + 4096 * kc, BOFF + 4096 * kc + 2048>(kr, k_base0, k_base1);
            float4_t S[2][2];
#pragma unroll
            for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    float4_t s = (float4_t){0.f, 0.f, 0.f, 0.f};
                    s = pf_mfma(__builtin_bit_cast(half8_t, kr[2 * kb2]), qop[rb][0], s);
                    s = pf_mfma(__builtin_bit_cast(half8_t, kr[2 * kb2 + 1]), qop[rb][1], s);
                    S[kb2][rb] = s;
                }
            }
            // masks, only where the chunk crosses some row's span boundary (uniform branch):
            // key j = j0 + 16*kb2 + 4g + i is outside row p's span [bp, p] iff
            // (j - bp) > (p - bp) as unsigned
            if (j0 + 31u > w_pmin || (a.n_swa && j0 < w_bmax)) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    const uint32_t p = row_pos[rb];
                    const uint32_t bp = a.n_swa ? (p + 1u > a.n_swa ? p + 1u - a.n_swa : 0u) : 0u;
                    const uint32_t off = j0 + 4u * g - bp, span = p - bp;
#pragma unroll
                    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (off + (16u * kb2 + i) > span) S[kb2][rb][i] = -INFINITY;
                }
            }
            // softmax weights per row block; P^T operand item i = key 16*(i/4) + 4g + i%4
            half8_t phi[2], plo[2];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                const float lmax = pf_max8(S[0][rb], S[1][rb]) * c;
                if (__builtin_amdgcn_ballot_w64(lmax > m_run[rb] + PF_RESCALE_SLACK) != 0) {
                    const float m_new = fmaxf(m_run[rb], pf_max16_32(lmax));
                    const float corr = __builtin_amdgcn_exp2f(m_run[rb] - m_new);
                    m_run[rb] = m_new;
                    Lsum[rb] *= corr;
#pragma unroll
                    for (int mb = 0; mb < 4; ++mb) O[mb][rb] *= corr;
                }
                const float bias = PF_LOG2_PSCALE - m_run[rb];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float ps = __builtin_amdgcn_exp2f(fmaf(S[i >> 2][rb][i & 3], c, bias));
                    const _Float16 hi = (_Float16) ps;
                    phi[rb][i] = hi;
                    if constexpr (SPLIT_P) plo[rb][i] = (_Float16) (ps - (float) hi);
                }
                Lsum[rb] = pf_mfma(ones, phi[rb], Lsum[rb]);
                if constexpr (SPLIT_P) Lsum[rb] = pf_mfma(ones, plo[rb], Lsum[rb]);
            }
            // P.V: V^T operands of channel blocks 2mp, 2mp + 1, each from two transposing reads
            pf_static_for<0, 2>([&](auto mp_c) {
                constexpr int mp = decltype(mp_c)::value;
                constexpr int VOFF = BOFF + (int) TILE_BYTES + 4096 * kc;
                u32x2_t vt[4];  // [h2 * 2 + (keys +16)]
                pf_read_vt<VOFF, VOFF + 2048>(vt, v_base[2 * mp], v_base[2 * mp + 1]);
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    const int mb = 2 * mp + h2;
                    const half8_t va = __builtin_bit_cast(
                        half8_t, (u32x4_t){vt[2 * h2][0], vt[2 * h2][1], vt[2 * h2 + 1][0], vt[2 * h2 + 1][1]});
#pragma unroll
                    for (int rb = 0; rb < 2; ++rb) {
                        O[mb][rb] = pf_mfma(va, phi[rb], O[mb][rb]);
                        if constexpr (SPLIT_P) O[mb][rb] = pf_mfma(va, plo[rb], O[mb][rb]);
                    }
                }
            });
        });
    };

    // ---- pipeline: tile kt in buffer kt & 1; tile kt + 1 is copied into the other buffer while
    // kt is computed
    auto step = [&](uint32_t kt, auto buf_c) {
        constexpr int BUF = decltype(buf_c)::value;
        __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of tile kt (and the next entries)
        __builtin_amdgcn_s_barrier();   // everyone's copies landed; everyone is done with kt - 1
        if (kt < kt_last) {
            copy_tile(kt + 1u, BUF ^ 1);
            if (kt + 1u < kt_last) load_pids(kt + 2u);
        }
        compute_tile(kt, buf_c);
    };
    load_pids(kt_first);
    copy_tile(kt_first, 0);
    if (kt_first < kt_last) load_pids(kt_first + 1u);
    for (uint32_t kt = kt_first; kt <= kt_last; kt += 2u) {
        step(kt, std::integral_constant<int, 0>{});
        if (kt + 1u <= kt_last) step(kt + 1u, std::integral_constant<int, 1>{});
    }

    // ---- finalise: the sink, the normalisation, the store -----------------------------------
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const float L = Lsum[rb][0];  // every lane of the row holds the row's sum
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
