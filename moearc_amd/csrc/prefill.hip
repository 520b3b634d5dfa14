// Chunked prefill over a paged f16 KV cache, head_dim 64, on gfx950 MFMA: the precise kernels
// (moearc_attn_prefill_precise_g{1,2,4,8}, softmax weights carried as f16 hi + lo), which the host
// selects when MOEARC_PREFILL_PRECISE=1 or when |scale * log2 e| > 1 (where the default kernels'
// f16 pre-scaled Q could leave f16's range); and the layout helpers the default kernels
// (prefill_fast.hip) share.
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
// Keys stream through LDS in 32-key tiles (one chunk each), four buffers, copies three tiles ahead:
// at the top of tile kt every wave waits for its copies of tile kt (a constant vmcnt: two copies
// and one block-table load per step) and meets the others at a barrier, issues the copies of tile
// kt + 3 into the buffer tile kt - 1 used, then computes tile kt. The copies are
// global_load_lds_dwordx4 (16 bytes per lane, placed at base + 16 * lane), so tiles go from the
// cache to LDS without passing through registers. Wave w copies keys 8w..8w+7 of each tile; when
// the tile lies in one page its block-table entry is wave-uniform and the copy takes one scalar
// base, otherwise every lane looks up its own key's page. Keys past the last query position are
// clamped to it, so no copy reads a slot the cache has not written.
//
// Matrix layout: v_mfma_f32_32x32x16_f16 throughout (on gfx950 it leaves room for a few VALU
// instructions beside each MFMA, where 16x16x32 leaves almost none). Per 32-key chunk a wave
//   S^T[32 keys x 32 rows] = K . Q^T            4 MFMAs (k = 16 channels each)
//   O^T[64 ch x 32 rows] += V^T . P^T           4 MFMAs (2 channel blocks x 2 steps of 16 keys)
// Lane (h, n) (h = lane / 32) holds S^T rows 8j + 4h + i (j, i = 0..3) of column n: 16 keys of
// query row n. Taken in register order, S regs 8s..8s+7 are exactly the k-slots 8h..8h+7 of the
// P^T operand of step s -- keys 16s + 4h + i and 16s + 8 + 4h + i -- so P needs no shuffles and V^T
// is read in that key order.
//
// LDS layout of a buffer: K and V each [64 keys][64 ch] f16, 128-byte rows whose 16-byte chunks are
// XOR-swizzled: chunk c of key k at k * 128 + ((c ^ f(k)) << 4). gfx950's LDS serves 256 bytes per
// clock from 64 banks (two 128-byte rows side by side); a ds_read_b128 is served in 16-lane passes
// that pair lanes i and i + 16, a 64-bit transposing read in 32-lane passes (as measured with
// SQ_LDS_BANK_CONFLICT). The swizzles keep every pass on distinct banks:
//   K: f(k) = (k & 7) ^ ((k >> 4) & 1) -- keys n and n + 16 of one pass differ in bit 4 only;
//   V: f(k) = (k & 7) ^ (((k >> 1) & 1) << 2) -- a half-wave reads 4 keys x 4 chunks, and the
//      term spreads them over both halves of the 8 chunk slots.
//   K operand of MFMA t: lane (h, m) takes channels 16t + 8h..+7 of key m -- one ds_read_b128.
//   V^T operand of (channel block mb, step s): lane (h, q, r) (q = lane / 16 & 1, r = lane & 15)
//      needs channel 32mb + 16q + r of keys 16s + 4h + j and 16s + 8 + 4h + j. ds_read_b64_tr_b16
//      transposes within each 16-lane group (lane r receives element r & 3 of the 8 bytes addressed
//      by lanes 4j + (r >> 2), j = 0..3), so lane r addresses key 16s + 4h + (r >> 2) (+8),
//      channels 32mb + 16q + 4(r & 3)..+3: two reads per operand.
// LDS reads are issued through asm with their waits: the compiler, which cannot tell the buffer
// being read from the one being filled by LDS DMA, would otherwise wait for the copy in flight
// before every read.
//
// Softmax. p = 2^(s*c + 7 - m) in the log2 domain (c = scale * log2 e) against a per-row reference
// m that moves only when some weight of the row overflows f16 (a score more than ~9 above m): the
// weights are computed first, an infinite row sum flags the overflow, and only then are the
// cross-lane row maximum, the rescale of O and the sums and the recomputation run (in practice at
// a row's first chunk). So p < 2^16 fits f16, and the common chunk computes no maximum. p is split
// p = p_hi + p_lo into two f16 MFMA operands (~22 bits, like the decode kernel), so prefill rows
// equal decode calls to ~2e-7; the row sums are dot products of the same f16 parts with ones
// (v_dot2_f32_f16), so numerator and denominator see the same rounding. Causal/window masks are
// applied only in chunks that cross a row's span boundary.
#include "common.h"

#define PF_LOG2_PSCALE 7.0f
#define PF_M_INIT -1.0e30f  // finite "no key yet": keeps exp2(m_old - m_new) defined for rows
                            // whose keys all lie in later chunks
#define PF_KT 32            // keys per LDS tile (one chunk)
#define PF_NBUF 4           // tile buffers in LDS: copies run PF_NBUF - 1 tiles ahead

typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float16_t pf_mfma(const half8_t a, const half8_t b, const float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Byte offset of 16-byte chunk c (8 channels) of key k within a K tile ...
__device__ __forceinline__ uint32_t k_swz(uint32_t k) { return (k & 7u) ^ ((k >> 4) & 1u); }
__device__ __forceinline__ uint32_t k_off(uint32_t k, uint32_t c) {
    return k * 128u + ((c ^ k_swz(k)) << 4);
}

// ... and within a V tile.
__device__ __forceinline__ uint32_t v_swz(uint32_t k) { return (k & 7u) ^ (((k >> 1) & 1u) << 2); }
__device__ __forceinline__ uint32_t v_off(uint32_t k, uint32_t c) {
    return k * 128u + ((c ^ v_swz(k)) << 4);
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, typename F>
__device__ __forceinline__ void pf_static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        pf_static_for<B + 1, E>(f);
    }
}

// K operands of one chunk: r[t] at base[t] + O (channels 16t + 8h..+7 of key m).
template <int O>
__device__ __forceinline__ void pf_read_k(u32x4_t (&r)[4], const uint32_t (&base)[4]) {
    asm volatile(
        "ds_read_b128 %0, %4 offset:%8\n\t"
        "ds_read_b128 %1, %5 offset:%8\n\t"
        "ds_read_b128 %2, %6 offset:%8\n\t"
        "ds_read_b128 %3, %7 offset:%8\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(base[0]), "v"(base[1]), "v"(base[2]), "v"(base[3]), "i"(O)
        : "memory");
}

// V^T operands of one channel block: r[2s + e] = keys 16s + 8e + 4h + (0..3), by transposing reads.
template <int O>
__device__ __forceinline__ void pf_read_vt(u32x2_t (&r)[4], uint32_t base) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %4 offset:%5\n\t"
        "ds_read_b64_tr_b16 %1, %4 offset:%6\n\t"
        "ds_read_b64_tr_b16 %2, %4 offset:%7\n\t"
        "ds_read_b64_tr_b16 %3, %4 offset:%8\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(base), "i"(O), "i"(O + 1024), "i"(O + 2048), "i"(O + 3072)
        : "memory");
}

// LDS DMA of 16 bytes per lane from a wave-uniform global base plus a per-lane 32-bit offset to
// LDS address lds + 16 * lane (the scalar-base form: no 64-bit address arithmetic per lane).
__device__ __forceinline__ void pf_copy16(const void *sbase, uint32_t voff, uint32_t lds) {
    // M0 is read by the DMA one wait state after it is written; it is the compiler's register, so
    // the statement saves it first and restores it after the DMA has issued (no m0 clobber)
    uint32_t m0_saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(m0_saved) : "v"(voff), "s"(sbase), "s"(lds) : "memory");
}

template <int GROUP>
__device__ __forceinline__ void prefill_body(const PrefillArgs &a) {
    constexpr uint32_t ROWS = MOEARC_PREFILL_ROWS;  // 128 rows per work-group
    constexpr uint32_t TOK = ROWS / GROUP;          // query tokens per work-group
    constexpr uint32_t TILE_BYTES = PF_KT * 128u;   // one K or V tile
    constexpr uint32_t BUF_BYTES = 2u * TILE_BYTES;  // K tile, V tile
    __shared__ __attribute__((aligned(1024))) uint8_t tiles[PF_NBUF * BUF_BYTES];

    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t G = a.n_kv_heads;
    const uint32_t kvh = blockIdx.x % G;
    const uint32_t qt = a.n_qtiles - 1u - blockIdx.x / G;
    const uint32_t q0 = qt * TOK;                   // first query token of the work-group
    const uint32_t q_end = min(q0 + TOK, a.n_q);
    const uint32_t h = lane >> 5, n = lane & 31u;
    const uint32_t sh = a.pt_shift, pmask = (1u << sh) - 1u;

    // key span of the whole work-group
    const uint32_t p_first = a.pos0 + q0, p_last = a.pos0 + q_end - 1u;
    const uint32_t k_lo = a.n_swa ? (p_first + 1u > a.n_swa ? p_first + 1u - a.n_swa : 0u) : 0u;
    const uint32_t kt_first = k_lo / PF_KT, kt_last = p_last / PF_KT;

    // ---- this lane's query row: local row n of the wave -> (token, head) -----------------------
    // Q^T operand of MFMA t: row n, channels 16t + 8h .. +7
    half8_t qop[4];
    const uint32_t r_wg = wave * 32u + n;
    const uint32_t tok = q0 + r_wg / GROUP, hd = kvh * GROUP + r_wg % GROUP;
    const bool row_ok = tok < q_end;
    const uint32_t row_pos = a.pos0 + min(tok, q_end - 1u);
    const uint32_t row_bp = a.n_swa ? (row_pos + 1u > a.n_swa ? row_pos + 1u - a.n_swa : 0u) : 0u;
    {
        const uint16_t *src = a.q + ((uint64_t) min(tok, a.n_q - 1u) * a.n_heads + hd) * 64u + 8u * h;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            u32x4_t v = *(const u32x4_t *) (src + 16 * t);
            if (!row_ok) v = (u32x4_t){0u, 0u, 0u, 0u};
            qop[t] = __builtin_bit_cast(half8_t, v);
        }
    }
    // the wave's position range, for deciding which chunks need masks
    const uint32_t w_tok0 = q0 + (wave * 32u) / GROUP;
    const uint32_t w_tok1 = min(q0 + (wave * 32u + 31u) / GROUP, q_end - 1u);
    const uint32_t w_pmin = a.pos0 + min(w_tok0, q_end - 1u), w_pmax = a.pos0 + w_tok1;
    const uint32_t w_bmin = a.n_swa ? (w_pmin + 1u > a.n_swa ? w_pmin + 1u - a.n_swa : 0u) : 0u;
    const uint32_t w_bmax = a.n_swa ? (w_pmax + 1u > a.n_swa ? w_pmax + 1u - a.n_swa : 0u) : 0u;

    float c = a.scale_log2e;
    // s*c with c < 0 equals (-s)*(-c): negate the f16 Q operand (exact) so that c > 0 and the row
    // maximum of s*c is c times the maximum of s
    if (c < 0.f) {
        c = -c;
#pragma unroll
        for (int t = 0; t < 4; ++t) qop[t] = -qop[t];
    }
    float m_run = PF_M_INIT;
    float l_run = 0.f;  // this lane's share of the row sum (its 16 keys of every chunk)
    float16_t O[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) O[mb][i] = 0.f;

    // ---- per-lane LDS base addresses (buffer 0, chunk 0, tile offset excluded) ----------------
    const uint32_t lds0 = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) uint8_t *) tiles;
    uint32_t k_base[4], v_base[2];
#pragma unroll
    for (int t = 0; t < 4; ++t) k_base[t] = lds0 + k_off(n, 2u * t + h);
    {
        const uint32_t r = lane & 15u, q = (lane >> 4) & 1u;
        const uint32_t vkey = 4u * h + (r >> 2);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
            v_base[mb] = lds0 + v_off(vkey, 4u * mb + 2u * q + ((r >> 1) & 1u)) + ((r & 1u) << 3);
    }

    // ---- tile copies: lane L of wave w fills LDS chunk slot L & 7 of key k = 8w + (L >> 3) of the
    // K and the V tile; that slot holds chunk (L & 7) ^ f(k) of the key.
    const uint32_t ld_key = 8u * wave + (lane >> 3);
    const uint32_t ld_chunk = (lane & 7u) ^ k_swz(ld_key), ld_chunk_v = (lane & 7u) ^ v_swz(ld_key);
    const uint64_t row_bytes = (uint64_t) G * 128u;
    const uint32_t lane_ck = kvh * 128u + ld_chunk * 16u, lane_cv = kvh * 128u + ld_chunk_v * 16u;
    // Block-table entry of this lane's key of tile kt (keys past p_last are clamped to it, so no copy
    // reads a slot the cache has not written), issued through asm: the pipeline below waits for it
    // explicitly, and the compiler's own tracking would add conservative waits in the loop.
    auto key_of = [&](uint32_t kt) { return min(kt * PF_KT + ld_key, p_last); };
    auto load_pid = [&](uint32_t kt) -> uint32_t {
        const uint32_t *p = a.block_table + (key_of(kt) >> sh);
        uint32_t v;
        asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p) : "memory");
        return v;
    };
    // A tile that lies wholly below p_last in pages of 32 keys or more sits in one page: its base
    // row is wave-uniform and computed on the scalar unit, and each lane adds a fixed 32-bit offset
    // (VALU issue is the scarce resource beside the MFMAs). Other tiles address per lane.
    const bool uni_pages = sh >= 5u;
    const uint32_t lane_k = ld_key * (uint32_t) row_bytes + lane_ck;
    const uint32_t lane_v = ld_key * (uint32_t) row_bytes + lane_cv;
    auto copy_tile = [&](uint32_t kt, uint32_t pid, int buf) {
        uint8_t *dst = tiles + buf * BUF_BYTES + 8u * wave * 128u;
        if (uni_pages && kt * PF_KT + (PF_KT - 1u) <= p_last) {
            const uint32_t pid0 = __builtin_amdgcn_readfirstlane(pid);
            const uint64_t base = (((uint64_t) pid0 << sh) | ((kt * PF_KT) & pmask)) * row_bytes;
            const uint32_t lds = __builtin_amdgcn_readfirstlane(
                (uint32_t) (uintptr_t) (__attribute__((address_space(3))) uint8_t *) dst);
            pf_copy16((const uint8_t *) a.k_pages + base, lane_k, lds);
            pf_copy16((const uint8_t *) a.v_pages + base, lane_v, lds + TILE_BYTES);
        } else {
            const uint64_t off = (uint64_t) ((pid << sh) | (key_of(kt) & pmask)) * row_bytes;
            __builtin_amdgcn_global_load_lds((const uint8_t *) a.k_pages + off + lane_ck, dst, 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const uint8_t *) a.v_pages + off + lane_cv, dst + TILE_BYTES, 16, 0, 0);
        }
    };

    // ---- chunk stages ----------------------------------------------------------------------------
    const half2_t ones2 = {1, 1};
    // QK^T of chunk kc of the tile in buffer offset BOFF: S reg 4j + i = key j0 + 8j + 4h + i of row n
    auto qk = [&](auto boff_c, auto kc_c, const float16_t &init) -> float16_t {
        constexpr int BOFF = decltype(boff_c)::value, kc = decltype(kc_c)::value;
        u32x4_t kr[4];
        pf_read_k<BOFF + 4096 * kc>(kr, k_base);
        float16_t S = init;
#pragma unroll
        for (int t = 0; t < 4; ++t) S = pf_mfma(__builtin_bit_cast(half8_t, kr[t]), qop[t], S);
        return S;
    };
    // masks for chunk keys j0..j0+31: key j is outside the row's span [bp, p] iff
    // (j - bp) > (p - bp) as unsigned
    auto mask = [&](float16_t &S, uint32_t j0) {
        const uint32_t off = j0 + 4u * h - row_bp, span = row_pos - row_bp;
#pragma unroll
        for (int i = 0; i < 16; ++i)
            if (off + (uint32_t) (8 * (i >> 2) + (i & 3)) > span) S[i] = -INFINITY;
    };
    // softmax weights; P^T operand of step s = S regs 8s..8s+7 in order. Returns l0 plus this
    // lane's share of the chunk's row sum: f16 weights summed with ones (v_dot2_f32_f16), so the
    // denominator sees the same rounding as the numerator. Weights are non-negative, so the sum
    // is finite unless some weight overflowed f16 (became +inf).
    auto weights = [&](const float16_t &S, float bias, float l0, half8_t (&phi)[2], half8_t (&plo)[2]) {
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const float x0 = fmaf(S[i], c, bias);
            const float x1 = fmaf(S[i + 1], c, bias);
            const float p0 = __builtin_amdgcn_exp2f(x0);
            const float p1 = __builtin_amdgcn_exp2f(x1);
            const half2_t hv = {(_Float16) p0, (_Float16) p1};
            phi[i >> 3][i & 7] = hv[0];
            phi[i >> 3][(i & 7) + 1] = hv[1];
            l0 = __builtin_amdgcn_fdot2(hv, ones2, l0, false);
            const half2_t lv = {(_Float16) (p0 - (float) hv[0]), (_Float16) (p1 - (float) hv[1])};
            plo[i >> 3][i & 7] = lv[0];
            plo[i >> 3][(i & 7) + 1] = lv[1];
        }
        return l0;
    };
    auto lo_sum = [&](const half8_t (&plo)[2], float l0) {
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int i = 0; i < 8; i += 2)
                l0 = __builtin_amdgcn_fdot2((half2_t){plo[s2][i], plo[s2][i + 1]}, ones2, l0, false);
        return l0;
    };
    // The reference m_run is not compared with the chunk's maximum up front. The weights are
    // computed against it directly; a score more than ~9 above it (or any visible key of a row
    // that has seen none) yields a weight >= 2^16, which overflows f16 and makes the lane's sum
    // infinite. Only then is the row maximum taken, the reference moved (O and l rescaled) and
    // the weights recomputed, so weights stay below 2^16 and the common chunk pays no max.
    auto softmax = [&](float16_t &S, half8_t (&phi)[2], half8_t (&plo)[2]) {
        float l_new = weights(S, PF_LOG2_PSCALE - m_run, l_run, phi, plo);
        if (__builtin_amdgcn_ballot_w64(l_new == INFINITY) != 0) {
            const float16_t R = S * c;
            float lmax = fmaxf(R[0], R[1]);
#pragma unroll
            for (int i = 2; i < 16; i += 2) lmax = fmaxf(lmax, fmaxf(R[i], R[i + 1]));
            const float m_new = fmaxf(m_run, fmaxf(lmax, __shfl_xor(lmax, 32)));
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= corr;
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) O[mb] *= corr;
            l_new = weights(S, PF_LOG2_PSCALE - m_run, l_run, phi, plo);
        }
        l_new = lo_sum(plo, l_new);
        l_run = l_new;
    };
    // P.V per channel block: operands of steps 0, 1 from four transposing reads
    auto pv = [&](auto boff_c, auto kc_c, const half8_t (&phi)[2], const half8_t (&plo)[2]) {
        constexpr int BOFF = decltype(boff_c)::value, kc = decltype(kc_c)::value;
        pf_static_for<0, 2>([&](auto mb_c) {
            constexpr int mb = decltype(mb_c)::value;
            u32x2_t vt[4];
            pf_read_vt<BOFF + (int) TILE_BYTES + 4096 * kc>(vt, v_base[mb]);
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const half8_t va = __builtin_bit_cast(
                    half8_t, (u32x4_t){vt[2 * s][0], vt[2 * s][1], vt[2 * s + 1][0], vt[2 * s + 1][1]});
                O[mb] = pf_mfma(va, phi[s], O[mb]);
                O[mb] = pf_mfma(va, plo[s], O[mb]);
            }
        });
    };

    // ---- one tile (= one chunk): skipped when no row of the wave sees it, masked when it crosses
    // some row's span boundary (uniform branches)
    auto compute_tile = [&](uint32_t kt, auto boff_c) {
        const uint32_t jc = kt * PF_KT;
        if (jc > w_pmax || jc + 31u < w_bmin) return;
        using K0 = std::integral_constant<int, 0>;
        float16_t zero;
#pragma unroll
        for (int i = 0; i < 16; ++i) zero[i] = 0.f;
        const bool masked = jc + 31u > w_pmin || (a.n_swa && jc < w_bmax);
        float16_t S = qk(boff_c, K0{}, zero);
        if (masked) mask(S, jc);
        half8_t phi[2], plo[2];
        softmax(S, phi, plo);
        pv(boff_c, K0{}, phi, plo);
    };

    // ---- pipeline over tiles kt_first + r, r = 0..nt-1, tile r in buffer r % PF_NBUF ------------
    // Per step r: wait until this wave's copies of tile r (and the block-table entry for tile r + 3)
    // have landed, meet the other waves (so every wave's copies of tile r are in, and every wave is
    // done with tile r - 1, whose buffer is reused), copy tile r + 3 into that buffer, load the entry
    // for tile r + 6, compute tile r. Indices past the last tile are clamped: those copies go to
    // buffers no later step reads, and every step issues the same three memory operations, so the
    // wait is a constant -- the six operations issued after the entry of tile r + 3 may be pending.
    const uint32_t nt = kt_last - kt_first + 1u;
    auto tile = [&](uint32_t r) { return kt_first + min(r, nt - 1u); };
    uint32_t pid[PF_NBUF];  // entries of tiles r + 3, r + 4, r + 5 (ring indexed by r % PF_NBUF)
    pid[0] = load_pid(tile(0));
    pid[1] = load_pid(tile(1));
    pid[2] = load_pid(tile(2));
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(pid[0]), "+v"(pid[1]), "+v"(pid[2]) : : "memory");
    copy_tile(tile(0), pid[0], 0);
    pid[3] = load_pid(tile(3));
    copy_tile(tile(1), pid[1], 1);
    pid[0] = load_pid(tile(4));
    copy_tile(tile(2), pid[2], 2);
    pid[1] = load_pid(tile(5));
    for (uint32_t r = 0; r < nt; r += PF_NBUF) {
        bool done = false;
        pf_static_for<0, PF_NBUF>([&](auto k_c) {
            constexpr int k = decltype(k_c)::value;
            if (done || r + k >= nt) {
                done = true;
                return;
            }
            // vmcnt(6), tied to the entry it makes valid so no use of it is scheduled above the wait
            asm volatile("s_waitcnt vmcnt(6)" : "+v"(pid[(k + 3) % PF_NBUF]) : : "memory");
            __builtin_amdgcn_s_barrier();
            copy_tile(tile(r + k + 3u), pid[(k + 3) % PF_NBUF], (k + 3) % PF_NBUF);
            pid[(k + 2) % PF_NBUF] = load_pid(tile(r + k + 6u));
            compute_tile(tile(r + k), std::integral_constant<int, k * (int) BUF_BYTES>{});
        });
    }
    // The clamped copies past the last tile may still be in flight: they must land before this
    // work-group's LDS is released. The block-table loads of the last steps are in flight too;
    // the wait names their registers so that none is given to another value before they land
    // (an asm load's destination is written whenever the data arrives).
    asm volatile("s_waitcnt vmcnt(0)"
                 : "+v"(pid[0]), "+v"(pid[1]), "+v"(pid[2]), "+v"(pid[3])
                 :
                 : "memory");
    __builtin_amdgcn_s_waitcnt(0);

    // ---- finalise: row sum over the lane pair, the sink, the normalisation, the store ---------
    const float L = l_run + __shfl_xor(l_run, 32);
    const float sink2 = a.sinks ? a.sinks[hd] * MOEARC_LOG2E : -INFINITY;
    const float Mt = fmaxf(m_run, sink2);
    const float fm = __builtin_amdgcn_exp2f(m_run - Mt);
    const float inv = fm / (L * fm + __builtin_amdgcn_exp2f(sink2 - Mt + PF_LOG2_PSCALE));
    if (row_ok) {
        const uint64_t o = ((uint64_t) tok * a.n_heads + hd) * 64u;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // O reg 4j + i = channel 32mb + 8j + 4h + i of row n
                const float4_t v = {O[mb][4 * j] * inv, O[mb][4 * j + 1] * inv, O[mb][4 * j + 2] * inv,
                                    O[mb][4 * j + 3] * inv};
                const uint32_t d = 32u * mb + 8u * j + 4u * h;
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

// The precise kernels (p split into f16 hi + lo); the default single-f16 kernels are in
// prefill_fast.hip.
#define PREFILL_KERNEL(GRP)                                                                      \
    extern "C" __global__ __launch_bounds__(MOEARC_PREFILL_THREADS) void                        \
        moearc_attn_prefill_precise_g##GRP(const PrefillArgs a) {                                \
        prefill_body<GRP>(a);                                                              \
    }

PREFILL_KERNEL(1)
PREFILL_KERNEL(2)
PREFILL_KERNEL(4)
PREFILL_KERNEL(8)
