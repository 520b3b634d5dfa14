// Rotary position embedding (NeoX or adjacent-pair convention, YaRN context extension), and the
// same rotation fused into the f16 K/V append of a prefill chunk.
//
// Semantics are moearc_rope's (kernels.cpp:1385-1468), which follow ggml's rope_yarn: for pair
// index p (channels (p, p + n_dims/2) with NeoX, (2p, 2p + 1) otherwise),
//   theta_extrap = pos * theta_scale^p,   theta_scale = freq_base^(-2/n_dims) (computed on the host)
//   theta        = freq_scale * theta_extrap
//   with YaRN (ext_factor != 0):  ramp  = 1 - clamp((p - corr_lo) / max(0.001, corr_hi - corr_lo), 0, 1)
//                                 theta = theta * (1 - ramp*ext) + theta_extrap * ramp*ext
//                                 mscale = attn_factor * (1 + 0.1 ln(1/freq_scale))
//   (x0, x1) -> (x0 cos - x1 sin, x0 sin + x1 cos) * mscale
// Channels at or above n_dims pass through unchanged. The angle is the closed form (each thread
// independent), as the reference's kernel computes it; cos and sin are the accurate library
// functions (full range reduction), since positions reach 10^5 radians.
//
// One thread per (token, pair, group of heads): it computes the angle once and writes both channels
// of the pair in each of its heads -- for the fused append, of K (rotated) and V (copied), as f16
// with the reference's rounding.
#include "common.h"

// f32_to_f16_bits: kernels_misc.hip (same translation unit).

// Rotation factors (cos, sin, both scaled by mscale) of pair p at position pos.
__device__ __forceinline__ float2_t rope_factors(const RopeParams &r, int pos, uint32_t p) {
    const float theta_extrap = (float) pos * powf(r.theta_scale, (float) p);
    float theta = r.freq_scale * theta_extrap;
    float mscale = r.attn_factor;
    if (r.ext_factor != 0.0f) {
        const float y = ((float) p - r.corr_lo) / fmaxf(0.001f, r.corr_hi - r.corr_lo);
        const float ramp_mix = (1.0f - fminf(1.0f, fmaxf(0.0f, y))) * r.ext_factor;
        theta = theta * (1.0f - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / r.freq_scale);
    }
    float s, c;
    sincosf(theta, &s, &c);
    return (float2_t){c * mscale, s * mscale};
}

// The rotation of one pair, (x0, x1) -> (x0 cos - x1 sin, x0 sin + x1 cos), with the roundings
// fixed by explicit fmas: every kernel here uses this one expression, so that the fused append and
// the separate rope + append paths agree to the bit whatever the compiler would contract.
__device__ __forceinline__ void rope_rotate(float x0, float x1, float2_t cs, float &o0, float &o1) {
    o0 = fmaf(x0, cs[0], -(x1 * cs[1]));
    o1 = fmaf(x0, cs[1], x1 * cs[0]);
}

// Channels (lo, hi) handled by pair slot j of a head_dim-wide row: rotated pairs first, then the
// pass-through channels two at a time.
__device__ __forceinline__ void pair_channels(const RopeParams &r, uint32_t j, uint32_t &lo, uint32_t &hi) {
    const uint32_t half = r.n_dims >> 1;
    if (j < half) {
        lo = r.neox ? j : 2u * j;
        hi = r.neox ? j + half : 2u * j + 1u;
    } else {
        lo = r.n_dims + 2u * (j - half);
        hi = lo + 1u;
    }
}

// A thread handles ROPE_HEADS heads (launch_args.h). The angle depends on (position, pair) only,
// so a thread computes cos/sin once and applies them to ROPE_HEADS rows: the transcendental work
// shrinks by that factor, and the thread's 2*ROPE_HEADS independent loads (4*ROPE_HEADS when V
// rides along) are all issued before the first store.

// moearc_rope: src/dst f32 [n_tokens][n_heads][head_dim]; dst may equal src. F16: dst is written
// as binary16 (f32_to_f16_bits of the f32 result, as moearc_quantize_f16 would narrow it).
// Grid: x over (token, pair slot), y over groups of ROPE_HEADS heads.
template <bool F16>
__device__ __forceinline__ void rope_body(void *dst, const float *src, const int *pos, uint64_t n_tokens,
                                          uint32_t n_heads, uint32_t head_dim, const RopeParams &r) {
    const uint32_t slots = (head_dim + 1u) >> 1;  // pair slots per head (head_dim may be odd)
    const uint64_t g = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_tokens * slots) return;
    const uint32_t j = (uint32_t) (g % slots);
    const uint64_t t = g / slots;
    const uint32_t h0 = blockIdx.y * ROPE_HEADS;
    uint32_t lo, hi;
    pair_channels(r, j, lo, hi);
    const bool rot = j < (r.n_dims >> 1), has_hi = hi < head_dim;
    float x0[ROPE_HEADS] = {}, x1[ROPE_HEADS] = {};
#pragma unroll
    for (uint32_t i = 0; i < ROPE_HEADS; ++i) {
        if (h0 + i < n_heads) {
            const float *s = src + (t * n_heads + h0 + i) * head_dim;
            x0[i] = s[lo];
            x1[i] = has_hi ? s[hi] : 0.0f;
        }
    }
    float2_t cs = {1.0f, 0.0f};
    if (rot) cs = rope_factors(r, pos[t], j);
    auto put = [&](uint64_t at, float v) {
        if constexpr (F16) ((uint16_t *) dst)[at] = f32_to_f16_bits(v);
        else ((float *) dst)[at] = v;
    };
#pragma unroll
    for (uint32_t i = 0; i < ROPE_HEADS; ++i) {
        if (h0 + i < n_heads) {
            const uint64_t o = (t * n_heads + h0 + i) * head_dim;
            if (rot) {
                float o0, o1;
                rope_rotate(x0[i], x1[i], cs, o0, o1);
                put(o + lo, o0);
                put(o + hi, o1);
            } else {
                put(o + lo, x0[i]);
                if (has_hi) put(o + hi, x1[i]);
            }
        }
    }
}

extern "C" __global__ void moearc_rope_k(float *dst, const float *src, const int *pos, uint64_t n_tokens,
                                         uint32_t n_heads, uint32_t head_dim, RopeParams r) {
    rope_body<false>(dst, src, pos, n_tokens, n_heads, head_dim, r);
}
extern "C" __global__ void moearc_rope_f16_k(uint16_t *dst, const float *src, const int *pos, uint64_t n_tokens,
                                             uint32_t n_heads, uint32_t head_dim, RopeParams r) {
    rope_body<true>(dst, src, pos, n_tokens, n_heads, head_dim, r);
}

// A prefill chunk's K (rotated) and V to (page_ids[t], slots[t]); k, v f32 [n_tok][n_kv_heads][head_dim].
// A slot outside the page is not written and is recorded in *err, as in moearc_kv_append_chunk.
// Grid as moearc_rope_k's.
extern "C" __global__ void moearc_rope_kv_append_chunk_k(void *k_pages, void *v_pages, const float *k,
                                                         const float *v, const int *pos,
                                                         const uint32_t *page_ids, const uint32_t *slots,
                                                         uint64_t n_tok, uint32_t n_kv_heads,
                                                         uint32_t head_dim, uint64_t page_tokens,
                                                         uint32_t kv_type, RopeParams r, uint32_t *err) {
    const uint32_t nslot = (head_dim + 1u) >> 1;
    const uint64_t g = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_tok * nslot) return;
    const uint32_t j = (uint32_t) (g % nslot);
    const uint64_t t = g / nslot;
    const uint32_t h0 = blockIdx.y * ROPE_HEADS;
    uint32_t lo, hi;
    pair_channels(r, j, lo, hi);
    const bool rot = j < (r.n_dims >> 1), has_hi = hi < head_dim;
    // Every load (rows, slot, page, position) is issued before the first use of any of them: one
    // memory latency instead of a chain of three.
    float k0[ROPE_HEADS] = {}, k1[ROPE_HEADS] = {}, v0[ROPE_HEADS] = {}, v1[ROPE_HEADS] = {};
#pragma unroll
    for (uint32_t i = 0; i < ROPE_HEADS; ++i) {
        if (h0 + i < n_kv_heads) {
            const uint64_t row = (t * n_kv_heads + h0 + i) * head_dim;
            k0[i] = k[row + lo];
            v0[i] = v[row + lo];
            k1[i] = has_hi ? k[row + hi] : 0.0f;
            v1[i] = has_hi ? v[row + hi] : 0.0f;
        }
    }
    const uint32_t slot = slots[t], page = page_ids[t];
    const int p = pos[t];
    asm volatile("" ::"v"(page), "v"(p));  // keeps the two loads above the branch
    if (slot >= page_tokens) {
        if (j == 0) *(volatile uint32_t *) err = 1u;  // every writer stores the same value
        return;
    }
    if (rot) {
        const float2_t cs = rope_factors(r, p, j);
#pragma unroll
        for (uint32_t i = 0; i < ROPE_HEADS; ++i) rope_rotate(k0[i], k1[i], cs, k0[i], k1[i]);
    }
    const uint64_t base = ((uint64_t) page * page_tokens + slot) * n_kv_heads;
#pragma unroll
    for (uint32_t i = 0; i < ROPE_HEADS; ++i) {
        if (h0 + i < n_kv_heads) {
            const uint64_t dst = (base + h0 + i) * head_dim;
            if (kv_type == MOEARC_KV_F16) {
                uint16_t *kp = (uint16_t *) k_pages + dst, *vp = (uint16_t *) v_pages + dst;
                kp[lo] = f32_to_f16_bits(k0[i]);
                vp[lo] = f32_to_f16_bits(v0[i]);
                if (has_hi) {
                    kp[hi] = f32_to_f16_bits(k1[i]);
                    vp[hi] = f32_to_f16_bits(v1[i]);
                }
            } else {
                float *kp = (float *) k_pages + dst, *vp = (float *) v_pages + dst;
                kp[lo] = k0[i];
                vp[lo] = v0[i];
                if (has_hi) {
                    kp[hi] = k1[i];
                    vp[hi] = v1[i];
                }
            }
        }
    }
}

// The fused append for the common geometry -- NeoX pairs over all 64 channels (n_dims = head_dim =
// 64), f16 pools, n_kv_heads dividing 16. A work-group covers 16 (token, KV head) rows, 16 /
// n_kv_heads whole tokens; lane c of a row's 16 holds channels 4c .. 4c + 3 of K and of V (one
// 16-byte load each: whole rows per load instruction). Pair p = 4 (c & 7) + i has its halves in
// lanes c and c ^ 8, which trade their K values (__shfl_xor by 8; a DPP row rotation built with
// __builtin_amdgcn_update_dpp here read element 0's register for all four elements); the cos and sin
// of each (token, pair) are computed once per work-group into LDS (the generic kernel computes
// them once per 4 heads). Each lane stores 8 bytes of K and of V -- a row is one 128-byte line --
// written through to the device-coherent level. Same results as moearc_rope_kv_append_chunk_k.
//
// sx = px[0 .. 3] summed over n >= 1 slices `stride` floats apart, in slice order (and sv the same
// of pv when TWO): per element the additions, in the order, of moearc_matmul_reduce_k, so with its
// bias added after them the values equal what it stores for a chunk product's split-K sums. Eight
// slices' loads of both rows leave before the first add (one memory round trip for up to 8).
template <bool TWO>
__device__ __forceinline__ void slice_sums4(const float *px, const float *pv, uint64_t stride, uint32_t n,
                                            float4_t &sx, float4_t &sv) {
    for (uint32_t z = 0; z < n; z += 8u) {
        float4_t a[8], b[8];
#pragma unroll
        for (uint32_t k = 0; k < 8u; ++k) {
            const uint64_t o = (uint64_t) min(z + k, n - 1u) * stride;
            a[k] = *(const float4_t *) (px + o);
            if constexpr (TWO) b[k] = *(const float4_t *) (pv + o);
        }
#pragma unroll
        for (uint32_t k = 0; k < 8u; ++k) {
            sx = z + k == 0u ? a[k] : z + k < n ? sx + a[k] : sx;
            if constexpr (TWO) sv = z + k == 0u ? b[k] : z + k < n ? sv + b[k] : sv;
        }
    }
}

// Rows of 64 channels, 16 per work-group (row = (token, head) of n_heads rows per token, with
// n_heads dividing 16 or a multiple of 16, so the work-group's rows cover T <= 16 whole or
// partial tokens). KV: the rows are K (rotated) and V, appended at (page_ids[t], slots[t]); else
// the rows are q, rotated into q_out (binary16 when q_f16, f32 otherwise). SUMS: x and v are slice
// 0 of a chunk product's split-K sums (n_slices slices `stride` floats apart, [t][head * 64 + ch]
// in each), added here with the product's bias (bx, bv: [head * 64 + ch], or null) instead of being
// read as finished rows.
template <bool KV, bool SUMS = false>
__device__ __forceinline__ void rope64_rows(uint32_t b, uint32_t nh, const float *x, const float *v,
                                            void *q_out, uint32_t q_f16, uint16_t *k_pages,
                                            uint16_t *v_pages, const int *pos, const uint32_t *page_ids,
                                            const uint32_t *slots, uint64_t n_tok, uint64_t page_tokens,
                                            const RopeParams &r, uint32_t *err, float2_t *cs_tab,
                                            const float *bx = nullptr, const float *bv = nullptr,
                                            uint64_t stride = 0, uint32_t n_slices = 1) {
    const uint32_t tid = threadIdx.x, c = tid & 15u;
    // tokens the 16 rows touch: 16 / nh whole ones, or one (32-bit divisions only)
    const bool few = nh <= 16u;
    const uint32_t T = few ? 16u / nh : 1u;
    const uint64_t t_first = few ? (uint64_t) b * T : (uint64_t) (b / (nh >> 4));
    const uint64_t row = (uint64_t) b * 16u + (tid >> 4);
    const uint64_t t = few ? t_first + (tid >> 4) / nh : t_first;
    const bool live = t < n_tok;
    // this lane's pieces and its row's destination leave before anything waits on them
    float4_t kx = {}, vx = {};
    uint32_t slot = 0, page = 0;
    if (live) {
        if constexpr (SUMS) {
            if constexpr (KV) {  // before the sums, which wait on their loads
                slot = slots[t];
                page = page_ids[t];
            }
            const uint64_t bo = (row - t * nh) * 64u + 4u * c;
            const float4_t zero = {0.f, 0.f, 0.f, 0.f};
            const float4_t kb = bx ? *(const float4_t *) (bx + bo) : zero;
            float4_t vb = zero;
            if constexpr (KV) vb = bv ? *(const float4_t *) (bv + bo) : zero;
            slice_sums4<KV>(x + row * 64u + 4u * c, KV ? v + row * 64u + 4u * c : nullptr, stride, n_slices, kx, vx);
            if (bx) kx = kx + kb;
            if (KV && bv) vx = vx + vb;
        } else {
            kx = *(const float4_t *) (x + row * 64u + 4u * c);
            if constexpr (KV) vx = *(const float4_t *) (v + row * 64u + 4u * c);
        }
        if constexpr (KV && !SUMS) {
            slot = slots[t];
            page = page_ids[t];
        }
    }
    for (uint32_t i = tid; i < T * 32u; i += 256u) {
        const uint64_t tt = t_first + (i >> 5);
        if (tt < n_tok) cs_tab[i] = rope_factors(r, pos[tt], i & 31u);
    }
    __syncthreads();
    if (!live) return;  // whole rows leave together: the row exchange below stays within live rows
    if (KV && slot >= page_tokens) {
        if (c == 0) *(volatile uint32_t *) err = 1u;
        return;
    }
    const bool hi = c >= 8u;
    const uint32_t tl = (uint32_t) (t - t_first);
    float o[4];
    uint32_t ko[2], vo[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float kq = __shfl_xor(kx[i], 8);  // lane c ^ 8 of the same row
        const float2_t cs = cs_tab[tl * 32u + 4u * (c & 7u) + (uint32_t) i];
        float o0, o1;
        rope_rotate(hi ? kq : kx[i], hi ? kx[i] : kq, cs, o0, o1);
        o[i] = hi ? o1 : o0;
        const uint32_t kb = f32_to_f16_bits(o[i]), vb = f32_to_f16_bits(vx[i]);
        ko[i >> 1] = (i & 1) ? (ko[i >> 1] | (kb << 16)) : kb;
        vo[i >> 1] = (i & 1) ? (vo[i >> 1] | (vb << 16)) : vb;
    }
    if constexpr (KV) {
        const uint64_t dst = (((uint64_t) page * page_tokens + slot) * nh + (row - t * nh)) * 64u + 4u * c;
        store_through8(k_pages + dst, u32x2_t{ko[0], ko[1]});
        store_through8(v_pages + dst, u32x2_t{vo[0], vo[1]});
    } else if (q_f16) {
        store_through8((uint16_t *) q_out + row * 64u + 4u * c, u32x2_t{ko[0], ko[1]});
    } else {
        *(float4_t *) ((float *) q_out + row * 64u + 4u * c) = float4_t{o[0], o[1], o[2], o[3]};
    }
}

extern "C" __global__ void __launch_bounds__(256) moearc_rope_kv_append_chunk64_k(
    uint16_t *k_pages, uint16_t *v_pages, const float *k, const float *v, const int *pos,
    const uint32_t *page_ids, const uint32_t *slots, uint64_t n_tok, uint32_t n_kv_heads,
    uint64_t page_tokens, RopeParams r, uint32_t *err) {
    __shared__ float2_t cs_tab[16 * 32];
    rope64_rows<true>(blockIdx.x, n_kv_heads, k, v, nullptr, 0u, k_pages, v_pages, pos, page_ids, slots,
                      n_tok, page_tokens, r, err, cs_tab);
}

// RoPE of a chunk's q and the fused K/V append in one launch (the attention block's two steps
// between its projections and its attention, independent of each other): work-groups [0, nb_q)
// take q's rows, the rest K/V's, each as in rope64_rows. q f32 [n_tok][n_heads][64] -> q_out;
// results equal moearc_rope_f16_k (q_f16) or moearc_rope_k, and moearc_rope_kv_append_chunk64_k.
extern "C" __global__ void __launch_bounds__(256) moearc_rope_qkv_chunk64_k(
    void *q_out, const float *q, uint32_t n_heads, uint32_t q_f16, uint32_t nb_q,
    uint16_t *k_pages, uint16_t *v_pages, const float *k, const float *v, const int *pos,
    const uint32_t *page_ids, const uint32_t *slots, uint64_t n_tok, uint32_t n_kv_heads,
    uint64_t page_tokens, RopeParams r, uint32_t *err) {
    __shared__ float2_t cs_tab[16 * 32];
    if (blockIdx.x < nb_q)
        rope64_rows<false>(blockIdx.x, n_heads, q, nullptr, q_out, q_f16, nullptr, nullptr, pos, nullptr,
                           nullptr, n_tok, 0u, r, err, cs_tab);
    else
        rope64_rows<true>(blockIdx.x - nb_q, n_kv_heads, k, v, nullptr, 0u, k_pages, v_pages, pos, page_ids,
                          slots, n_tok, page_tokens, r, err, cs_tab);
}

// The same from a q/k/v chunk product's split-K sums, in place of its reduction launch: q, k and v
// point at slice 0 of each matrix's sums (n_slices >= 2 slices, part_stride floats apart), bq, bk
// and bv are the projections' biases (or null). Results equal moearc_matmul_reduce_k followed by
// moearc_rope_qkv_chunk64_k.
extern "C" __global__ void __launch_bounds__(256) moearc_rope_qkv_sums64_k(
    void *q_out, const float *q, uint32_t n_heads, uint32_t q_f16, uint32_t nb_q,
    uint16_t *k_pages, uint16_t *v_pages, const float *k, const float *v, const int *pos,
    const uint32_t *page_ids, const uint32_t *slots, uint64_t n_tok, uint32_t n_kv_heads,
    uint64_t page_tokens, RopeParams r, uint32_t *err, const float *bq, const float *bk, const float *bv,
    uint64_t part_stride, uint32_t n_slices) {
    __shared__ float2_t cs_tab[16 * 32];
    if (blockIdx.x < nb_q)
        rope64_rows<false, true>(blockIdx.x, n_heads, q, nullptr, q_out, q_f16, nullptr, nullptr, pos, nullptr,
                                 nullptr, n_tok, 0u, r, err, cs_tab, bq, nullptr, part_stride, n_slices);
    else
        rope64_rows<true, true>(blockIdx.x - nb_q, n_kv_heads, k, v, nullptr, 0u, k_pages, v_pages, pos,
                                page_ids, slots, n_tok, page_tokens, r, err, cs_tab, bk, bv, part_stride,
                                n_slices);
}
