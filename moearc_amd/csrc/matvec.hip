// Matrix-vector products against GGUF block-quantised weights -- the attention projections
// (attn.qkv, attn.proj: moe.rs:1942-1959, 2063-2071) -- and the f32 bias add after them.
//
// out[r] = sum_c W[r][c] * x[c] (+ bias[r]), W row-major, each row a whole number of blocks
// (kernels.cpp:1046-1111 single matrix, 1146-1200 batched). Formats: F32, F16, Q8_0, Q4_K, Q5_K,
// Q6_K, MXFP4, each decoded as ggml lays it out (reference.rs:168-300).
//
// HBM-bound: every weight byte is read once. The layout of the work:
//   * A lane owns the pieces lane, lane + 64, ... of a row (a piece is PE consecutive elements:
//     half a Q8_0 block, a K-quant sub-block, one MXFP4 block, 8 or 16 floats). The mapping is the
//     same for every row, so a lane loads the activation values of its pieces into registers once
//     and keeps them while the wave walks its rows; each row is one wave's, reduced across the
//     wave at the end, so the result does not depend on how rows are spread over waves or
//     launches (a batched launch is bit-identical to the single ones).
//   * Weight rows are staged through LDS: the wave copies the row's byte range with coalesced
//     16-byte loads of aligned granules (any alignment of W, any block size), then each lane
//     reads its pieces from LDS at byte granularity (aligned dword reads + v_alignbyte). The
//     next row's granules are in flight while the current one is decoded.
//   * The activation is staged once per work-group in LDS (padded so the per-lane reads of
//     pieces are bank-conflict free) and read into registers from there; when it does not fit,
//     each lane loads its values from global memory.
//   * Decoding uses the CDNA4 conversions directly: sign-extending byte converts (SDWA) for Q8_0,
//     v_cvt_f32_ubyte for the K-quant nibbles, v_cvt_scalef32_pk_f32_fp4 for MXFP4 (E2M1, two
//     elements per instruction) and mixed-precision FMAs for F16.
// Per-piece arithmetic: Q8_0 d * sum(q * x); MXFP4 2^(e-127) * sum(v * x); Q4_K/Q5_K
// d1 * sum(q * x) - m1 * sum(x); Q6_K (d * sc) * (sum(q * x) - 32 * sum(x)) -- the reference's
// per-element values regrouped by their common factors, within the reference's tolerance of
// 2 (n/32 + 5) u sum|w x| (kernels_gpu.rs:126-137).
#include "common.h"

namespace {

__device__ __forceinline__ uint32_t lds_u32(const uint8_t *L, uint32_t a) {
    return *(const uint32_t *) (L + a);
}
// The four bytes at any byte address.
__device__ __forceinline__ uint32_t lds_4(const uint8_t *L, uint32_t a) {
    const uint32_t b = a & ~3u;
    return __builtin_amdgcn_alignbyte(lds_u32(L, b + 4), lds_u32(L, b), a & 3u);
}
// The sixteen bytes at any byte address.
__device__ __forceinline__ u32x4_t lds_16(const uint8_t *L, uint32_t a) {
    const uint32_t b = a & ~3u, s = a & 3u;
    const uint32_t w0 = lds_u32(L, b), w1 = lds_u32(L, b + 4), w2 = lds_u32(L, b + 8);
    const uint32_t w3 = lds_u32(L, b + 12), w4 = lds_u32(L, b + 16);
    return u32x4_t{__builtin_amdgcn_alignbyte(w1, w0, s), __builtin_amdgcn_alignbyte(w2, w1, s),
                   __builtin_amdgcn_alignbyte(w3, w2, s), __builtin_amdgcn_alignbyte(w4, w3, s)};
}

// Sixteen bytes of global memory at a 16-byte aligned address.
__device__ __forceinline__ u32x4_t gload16(uintptr_t addr) {
    return *(const __attribute__((address_space(1))) u32x4_t *) addr;
}

__device__ __forceinline__ float f16_lo(uint32_t w) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) (w & 0xFFFFu));
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) (w >> 16));
}

// sum_j byte_j(w) * x[j] for the four unsigned bytes of w (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ float dot_u8x4(uint32_t w, const float *x, float s) {
    s = fmaf((float) (w & 0xFFu), x[0], s);
    s = fmaf((float) ((w >> 8) & 0xFFu), x[1], s);
    s = fmaf((float) ((w >> 16) & 0xFFu), x[2], s);
    return fmaf((float) (w >> 24), x[3], s);
}
// The same for signed bytes (sign-extending SDWA converts).
__device__ __forceinline__ float dot_i8x4(uint32_t w, const float *x, float s) {
    s = fmaf((float) (int8_t) w, x[0], s);
    s = fmaf((float) (int8_t) (w >> 8), x[1], s);
    s = fmaf((float) (int8_t) (w >> 16), x[2], s);
    return fmaf((float) (int8_t) (w >> 24), x[3], s);
}

// The (scale, min) pair of K-quant sub-block `is` from the 12 packed scale bytes at `a`
// (get_scale_min_k4, reference.rs:150-160): sub-blocks 0-3 keep 6-bit values in bytes is and
// is + 4; 4-7 split theirs between the low/high nibbles of byte is + 4 and the top two bits of
// bytes is - 4 and is.
__device__ __forceinline__ void scale_min_k4(const uint8_t *L, uint32_t a, uint32_t is, uint32_t &sc,
                                             uint32_t &m) {
    const uint32_t j = is & 3u;
    const uint32_t r0 = L[a + j], r1 = L[a + 4u + j], r2 = L[a + 8u + j];
    const bool lo = is < 4u;
    sc = lo ? (r0 & 63u) : ((r2 & 0xFu) | ((r0 >> 6) << 4));
    m = lo ? (r1 & 63u) : ((r2 >> 4) | ((r1 >> 6) << 4));
}

template <uint32_t TY> struct Fmt;

// F32: pieces of 8 floats (32 bytes). `valid` < PE only for a row's last, partial piece.
template <> struct Fmt<0> {
    static constexpr uint32_t PE = 8;
    static __device__ __forceinline__ float dot(const uint8_t *L, uint32_t a, uint32_t, const float *x,
                                                float, float acc, uint32_t valid) {
        u32x4_t u = lds_16(L, a), v = lds_16(L, a + 16u);
        uint32_t w[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        if (valid < PE) {
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) w[j] = j < valid ? w[j] : 0u;
        }
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) acc = fmaf(__uint_as_float(w[j]), x[j], acc);
        return acc;
    }
};

// F16: pieces of 16 halves (32 bytes).
template <> struct Fmt<1> {
    static constexpr uint32_t PE = 16;
    static __device__ __forceinline__ float dot(const uint8_t *L, uint32_t a, uint32_t, const float *x,
                                                float, float acc, uint32_t valid) {
        u32x4_t u = lds_16(L, a), v = lds_16(L, a + 16u);
        uint32_t w[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        if (valid < PE) {
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j)
                w[j] = 2u * j >= valid ? 0u : 2u * j + 1u == valid ? (w[j] & 0xFFFFu) : w[j];
        }
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            acc = fmaf(f16_lo(w[j]), x[2 * j], acc);
            acc = fmaf(f16_hi(w[j]), x[2 * j + 1], acc);
        }
        return acc;
    }
};

// Q8_0 (34-byte blocks: f16 d, 32 int8): piece k = half k of the block.
template <> struct Fmt<8> {
    static constexpr uint32_t PE = 16;
    static __device__ __forceinline__ float dot(const uint8_t *L, uint32_t a, uint32_t k, const float *x,
                                                float, float acc, uint32_t) {
        const float d = f16_lo(lds_4(L, a));
        const u32x4_t q = lds_16(L, a + 2u + 16u * k);
        float s = dot_i8x4(q.x, x, 0.f);
        s = dot_i8x4(q.y, x + 4, s);
        s = dot_i8x4(q.z, x + 8, s);
        s = dot_i8x4(q.w, x + 12, s);
        return fmaf(d, s, acc);
    }
};

// Q4_K (144-byte super-blocks of 256: f16 d, f16 dmin, 12 scale bytes, 128 nibble bytes): piece
// k = sub-block k, the low (k even) or high nibbles of qs[32 (k / 2) .. + 32].
template <> struct Fmt<12> {
    static constexpr uint32_t PE = 32;
    static __device__ __forceinline__ float dot(const uint8_t *L, uint32_t a, uint32_t k, const float *x,
                                                float xs, float acc, uint32_t) {
        const uint32_t dm = lds_4(L, a);
        uint32_t sc, m;
        scale_min_k4(L, a + 4u, k, sc, m);
        const float d1 = f16_lo(dm) * (float) sc, m1 = f16_hi(dm) * (float) m;
        const uint32_t sh = 4u * (k & 1u), qa = a + 16u + 32u * (k >> 1);
        const u32x4_t q0 = lds_16(L, qa), q1 = lds_16(L, qa + 16u);
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        float s = 0.f;
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) s = dot_u8x4((w[j] >> sh) & 0x0F0F0F0Fu, x + 4 * j, s);
        return fmaf(-m1, xs, fmaf(d1, s, acc));
    }
};

// Q5_K (176 bytes: d, dmin, 12 scale bytes, qh[32], qs[128]): piece k = sub-block k; the fifth
// bit of element l is bit k of qh[l].
template <> struct Fmt<13> {
    static constexpr uint32_t PE = 32;
    static __device__ __forceinline__ float dot(const uint8_t *L, uint32_t a, uint32_t k, const float *x,
                                                float xs, float acc, uint32_t) {
        const uint32_t dm = lds_4(L, a);
        uint32_t sc, m;
        scale_min_k4(L, a + 4u, k, sc, m);
        const float d1 = f16_lo(dm) * (float) sc, m1 = f16_hi(dm) * (float) m;
        const uint32_t sh = 4u * (k & 1u), qa = a + 48u + 32u * (k >> 1);
        const u32x4_t q0 = lds_16(L, qa), q1 = lds_16(L, qa + 16u);
        const u32x4_t h0 = lds_16(L, a + 16u), h1 = lds_16(L, a + 32u);
        const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        float s = 0.f;
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const uint32_t q = ((w[j] >> sh) & 0x0F0F0F0Fu) | (((h[j] >> k) & 0x01010101u) << 4);
            s = dot_u8x4(q, x + 4 * j, s);
        }
        return fmaf(-m1, xs, fmaf(d1, s, acc));
    }
};

// Q6_K (210 bytes: ql[128], qh[64], int8 scales[16], f16 d): piece k (16 elements) = half n = k/8,
// quarter c = (k/2) % 4, sixteen is = k % 2: low nibble (c < 2) or high nibble of
// ql[64n + 32 (c % 2) + 16 is ..], two bits 2c of qh[32n + 16 is ..], scale byte k.
template <> struct Fmt<14> {
    static constexpr uint32_t PE = 16;
    static __device__ __forceinline__ float dot(const uint8_t *L, uint32_t a, uint32_t k, const float *x,
                                                float xs, float acc, uint32_t) {
        const uint32_t n = k >> 3, c = (k >> 1) & 3u, is = k & 1u;
        const u32x4_t l = lds_16(L, a + 64u * n + 32u * (c & 1u) + 16u * is);
        const u32x4_t h = lds_16(L, a + 128u + 32u * n + 16u * is);
        const float ds = f16_lo(lds_4(L, a + 208u)) * (float) (int8_t) L[a + 192u + k];
        const uint32_t shl = 4u * (c >> 1), shh = 2u * c;
        const uint32_t lw[4] = {l.x, l.y, l.z, l.w}, hw[4] = {h.x, h.y, h.z, h.w};
        float s = 0.f;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t q = ((lw[j] >> shl) & 0x0F0F0F0Fu) | (((hw[j] >> shh) & 0x03030303u) << 4);
            s = dot_u8x4(q, x + 4 * j, s);
        }
        return fmaf(ds, fmaf(-32.f, xs, s), acc);
    }
};

// MXFP4 (17 bytes: E8M0 exponent e, 16 bytes of E2M1 pairs; element j in the low nibble of byte
// j, element j + 16 in the high one): one block per piece. Scale 2^(e - 127); exponents from 253
// up (where the reference's per-element products overflow f32) take the per-element form
// (kvalue * 2^(e-128)) * x.
template <> struct Fmt<39> {
    static constexpr uint32_t PE = 32;
    static __device__ __forceinline__ float dot(const uint8_t *L, uint32_t a, uint32_t, const float *x,
                                                float, float acc, uint32_t) {
        const uint32_t e = L[a];
        const u32x4_t q = lds_16(L, a + 1u);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        if (e < 253u) {
            float s = 0.f;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const float2_t v0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[j], 1.0f, 0);
                const float2_t v1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[j], 1.0f, 1);
                const float2_t v2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[j], 1.0f, 2);
                const float2_t v3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[j], 1.0f, 3);
                s = fmaf(v0.x, x[4 * j], s);
                s = fmaf(v0.y, x[4 * j + 16], s);
                s = fmaf(v1.x, x[4 * j + 1], s);
                s = fmaf(v1.y, x[4 * j + 17], s);
                s = fmaf(v2.x, x[4 * j + 2], s);
                s = fmaf(v2.y, x[4 * j + 18], s);
                s = fmaf(v3.x, x[4 * j + 3], s);
                s = fmaf(v3.y, x[4 * j + 19], s);
            }
            const float scale = __uint_as_float(e ? e << 23 : 0x00400000u);
            return fmaf(scale, s, acc);
        }
        const float half = __uint_as_float((e - 1u) << 23);
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
            for (uint32_t b = 0; b < 4; ++b) {
                const uint32_t byte = (w[j] >> (8 * b)) & 0xFFu;
                const float2_t v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(byte, 1.0f, 0);
                acc = fmaf((v.x * 2.0f) * half, x[4 * j + b], acc);
                acc = fmaf((v.y * 2.0f) * half, x[4 * j + b + 16], acc);
            }
        }
        return acc;
    }
};

constexpr bool needs_xsum(uint32_t ty) { return ty == 12 || ty == 13 || ty == 14; }

// v + the DPP-moved v (lanes the row mask leaves out add 0).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_add(float v) {
    const int moved = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
    return v + __int_as_float(moved);
}

// Sum over the 64 lanes, complete in lane 63: quad swaps, half-row and row mirrors (each lane of a
// 16-lane row then holds the row's sum), then row 0 -> 1 and 2 -> 3 (row_bcast:15) and row 1 ->
// 2, 3 (row_bcast:31).
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v = dpp_add<0xB1>(v);         // quad_perm [1,0,3,2]
    v = dpp_add<0x4E>(v);         // quad_perm [2,3,0,1]
    v = dpp_add<0x141>(v);        // row_half_mirror
    v = dpp_add<0x140>(v);        // row_mirror
    v = dpp_add<0x142, 0xA>(v);   // row_bcast:15
    return dpp_add<0x143, 0xC>(v);  // row_bcast:31
}

}  // namespace

extern __shared__ __attribute__((aligned(16))) uint8_t mv_smem[];

template <uint32_t TY, uint32_t PPL>
__device__ __forceinline__ void matvec_body(const MatvecArgs &a) {
    constexpr uint32_t BB = moearc_mv_bb(TY), BE = moearc_mv_be(TY), PE = Fmt<TY>::PE;
    static_assert(PE == moearc_mv_pe(TY), "piece size disagrees with the host table");
    constexpr uint32_t PPB = BE >= PE ? BE / PE : 1u;  // pieces per block
    constexpr uint32_t GMAX = moearc_mv_gmax(TY, PPL);
    constexpr uint32_t SP = 64u * PPL;                  // pieces per slab
    constexpr uint32_t XPAD = PE + 4u;                  // LDS floats per piece of the activation

    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    uint32_t seg = 0;
    while (seg + 1u < a.n_seg && blockIdx.x >= a.wg_end[seg]) ++seg;
    const uint32_t wg = blockIdx.x - (seg ? a.wg_end[seg - 1u] : 0u);
    const uint32_t rows = a.rows[seg], n_cols = a.n_cols, P = a.n_pieces, n_slabs = a.n_slabs;
    const float *x = a.x[seg];
    const uint8_t *W = a.w[seg];

    const uint32_t r0 = (wg * waves + wave) * a.rpw;
    const bool has_rows = r0 < rows;  // uniform per wave
    const uint32_t r1 = min(r0 + a.rpw, rows);
    const uint32_t units = has_rows ? (r1 - r0) * n_slabs : 0u;
    const uint32_t wb_off = a.x_lds_bytes + wave * a.wave_buf;
    uint8_t *wb = mv_smem + wb_off;

    // Byte offset of piece p's block (or of the piece itself, for F32/F16) within its row.
    auto piece_byte = [&](uint32_t p) -> uint64_t {
        return BE == 1u ? (uint64_t) p * (PE * BB) : (uint64_t) (p / PPB) * BB;
    };

    // Unit u = (row r0 + u / n_slabs, slab u % n_slabs). Two units' granules are in flight at
    // once, in registers ga / gb (a unit's LDS copy is written just before it is decoded).
    u32x4_t ga[GMAX], gb[GMAX];
    uint32_t da = 0, na = 0, db = 0, nb = 0;  // LDS offset of the first byte, granule count
    auto issue = [&](uint32_t u, u32x4_t (&g)[GMAX], uint32_t &delta, uint32_t &ng) {
        const uint32_t r = r0 + u / n_slabs, sl = u % n_slabs;
        const uint64_t b0 = piece_byte(sl * SP);
        const uint64_t b1 = min((uint64_t) a.row_bytes, piece_byte(min((sl + 1u) * SP, P) - 1u) +
                                                            (BE == 1u ? PE * BB : BB));
        const uintptr_t src = (uintptr_t) (W + (uint64_t) r * a.row_bytes + b0);
        const uintptr_t base = src & ~(uintptr_t) 15;
        delta = (uint32_t) (src - base);
        ng = (uint32_t) ((delta + (b1 - b0) + 15u) >> 4);  // >= 1: the host never launches P == 0
        // Every lane issues all GMAX loads (indices past the unit clamp to its last granule), so
        // the number of loads in flight is fixed and each LDS copy waits for its own only.
#pragma unroll
        for (uint32_t k = 0; k < GMAX; ++k) {
            const uint32_t gi = min(lane + 64u * k, ng - 1u);
            g[k] = gload16(base + 16u * (uintptr_t) gi);
        }
    };

    // The first row's weights are in flight before anything waits on the activation; the bias and
    // residual of the wave's rows (lane i: row r0 + i, at most 64 rows per wave) follow them, so
    // that no row waits for its own.
    const bool with_bias = (a.bias_mask >> seg) & 1u, with_res = (a.res_mask >> seg) & 1u;
    float bias_l = 0.f, res_l = 0.f;
    if (has_rows) {
        issue(0, ga, da, na);
        issue(min(1u, units - 1u), gb, db, nb);  // always two units in flight (re-reads past the end)
        if (lane < r1 - r0) {
            if (with_bias) bias_l = a.bias[seg][r0 + lane];
            if (with_res) res_l = a.out[seg][r0 + lane];
        }
    }
    if (a.x_in_lds) {  // activation -> LDS, piece p's values at floats [p * XPAD, p * XPAD + PE)
        constexpr uint32_t XB = 8;  // loads in flight per thread before their stores
        float *xl = (float *) mv_smem;
        const uint32_t total = P * PE;
        for (uint32_t c0 = threadIdx.x; c0 < total; c0 += XB * blockDim.x) {
            float v[XB];
#pragma unroll
            for (uint32_t k = 0; k < XB; ++k) {
                const uint32_t c = c0 + k * blockDim.x;
                v[k] = c < n_cols ? x[c] : 0.f;
            }
#pragma unroll
            for (uint32_t k = 0; k < XB; ++k) {
                const uint32_t c = c0 + k * blockDim.x;
                if (c < total) xl[(c / PE) * XPAD + c % PE] = v[k];
            }
        }
        __syncthreads();
    }
    if (!has_rows) return;

    float xr[PPL][PE];
    float xs[PPL];
    auto load_x = [&](uint32_t sl) {
#pragma unroll
        for (uint32_t i = 0; i < PPL; ++i) {
            const uint32_t p = sl * SP + lane + 64u * i;
            if (a.x_in_lds) {
                const float *xl = (const float *) mv_smem + (uint64_t) min(p, P - 1u) * XPAD;
#pragma unroll
                for (uint32_t j = 0; j < PE; j += 4) {
                    const float4_t v = *(const float4_t *) (xl + j);
                    xr[i][j] = v.x;
                    xr[i][j + 1] = v.y;
                    xr[i][j + 2] = v.z;
                    xr[i][j + 3] = v.w;
                }
            } else {
#pragma unroll
                for (uint32_t j = 0; j < PE; ++j) {
                    const uint64_t c = (uint64_t) min(p, P - 1u) * PE + j;
                    xr[i][j] = c < n_cols ? x[c] : 0.f;
                }
                // Drain here (vmcnt(0)): otherwise the compiler cannot tell these loads from the
                // weight granules in flight and waits for everything wherever xr is read.
                __builtin_amdgcn_s_waitcnt(0x0F70);
            }
            if constexpr (needs_xsum(TY)) {
                float t = 0.f;
#pragma unroll
                for (uint32_t j = 0; j < PE; ++j) t += xr[i][j];
                xs[i] = t;
            } else {
                xs[i] = 0.f;
            }
        }
    };

    float acc = 0.f;
    auto step = [&](uint32_t u, u32x4_t (&g)[GMAX], uint32_t &delta_ref, uint32_t &ng_ref) {
        const uint32_t sl = u % n_slabs, r = r0 + u / n_slabs;
        const uint32_t delta = delta_ref, ng = ng_ref;
#pragma unroll
        for (uint32_t k = 0; k < GMAX; ++k) {
            const uint32_t gi = lane + 64u * k;
            if (gi < ng) *(u32x4_t *) (wb + 16u * gi) = g[k];
        }
        issue(min(u + 2u, units - 1u), g, delta_ref, ng_ref);
        __builtin_amdgcn_wave_barrier();
        if (u == 0 || n_slabs > 1u) load_x(sl);
        const uint64_t slab_b0 = piece_byte(sl * SP);
#pragma unroll
        for (uint32_t i = 0; i < PPL; ++i) {
            const uint32_t p = sl * SP + lane + 64u * i;
            if (p < P) {
                const uint32_t at = wb_off + delta + (uint32_t) (piece_byte(p) - slab_b0);
                const uint32_t valid = BE == 1u ? min(PE, n_cols - p * PE) : PE;
                acc = Fmt<TY>::dot(mv_smem, at, p % PPB, xr[i], xs[i], acc, valid);
            }
        }
        __builtin_amdgcn_wave_barrier();
        if (sl + 1u == n_slabs) {
            acc = wave_sum_to_lane63(acc);
            const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 63));
            if (lane == r - r0) {  // the lane holding this row's bias and residual
                const float y = with_bias ? tot + bias_l : tot;
                a.out[seg][r] = with_res ? res_l + y : y;
            }
            acc = 0.f;
        }
    };
    for (uint32_t u = 0; u < units; u += 2u) {
        step(u, ga, da, na);
        if (u + 1u < units) step(u + 1u, gb, db, nb);
    }
}

#define MATVEC_KERNEL(NAME, TY, PPL)                                                              \
    extern "C" __global__ void __launch_bounds__(64 * MOEARC_MV_MAX_WAVES)                        \
        moearc_matvec_##NAME##_p##PPL(MatvecArgs a) {                                             \
        matvec_body<TY, PPL>(a);                                                                  \
    }

MATVEC_KERNEL(f32, 0, 1)
MATVEC_KERNEL(f32, 0, 2)
MATVEC_KERNEL(f32, 0, 4)
MATVEC_KERNEL(f16, 1, 1)
MATVEC_KERNEL(f16, 1, 2)
MATVEC_KERNEL(f16, 1, 4)
MATVEC_KERNEL(q8_0, 8, 1)
MATVEC_KERNEL(q8_0, 8, 2)
MATVEC_KERNEL(q8_0, 8, 4)
MATVEC_KERNEL(q4_k, 12, 1)
MATVEC_KERNEL(q4_k, 12, 2)
MATVEC_KERNEL(q4_k, 12, 4)
MATVEC_KERNEL(q5_k, 13, 1)
MATVEC_KERNEL(q5_k, 13, 2)
MATVEC_KERNEL(q5_k, 13, 4)
MATVEC_KERNEL(q6_k, 14, 1)
MATVEC_KERNEL(q6_k, 14, 2)
MATVEC_KERNEL(q6_k, 14, 4)
MATVEC_KERNEL(mxfp4, 39, 1)
MATVEC_KERNEL(mxfp4, 39, 2)
MATVEC_KERNEL(mxfp4, 39, 4)

// out[i] = a[i] + b[i] (kernels.cpp:1676-1683); out may alias a or b (each index reads its own).
extern "C" __global__ void moearc_add_k(float *out, const float *x, const float *y, uint64_t n) {
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t) gridDim.x * blockDim.x)
        out[i] = x[i] + y[i];
}
