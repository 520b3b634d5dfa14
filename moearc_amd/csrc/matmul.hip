// Chunk-form projections on MFMA: Y[t][r] = sum_c W[r][c] X[t][c] (+ bias[r]) for the tokens of a
// prompt chunk -- the GEMM that the reference's prefill performs as one matvec per token
// (moe.rs:1942-1959, 2063-2071; kernels.cpp:1046-1111), W in Q8_0 or F16.
//
// Precision matches the matvec path, not f16 arithmetic: X is split into f16 hi + lo
// (x - hi - lo <= 2^-22 |x|), the Q8_0 payload enters the MFMA as exact f16 integers, each
// 32-wide block's f32 sum q . (hi + lo) comes from two chained v_mfma_f32_16x16x32_f16 and is
// scaled by the block's d in f32. F16 weights enter as they are. Activations must stay below
// 65504 in magnitude (the f16 range of the hi part).
//
// Work-group: 4 waves x RT 16-row tiles, 64 tokens (four 16x16 MFMA tiles per row tile): each
// activation fragment a wave loads feeds all of its row tiles. Operand
// layouts (16x16x32 f16): lane l holds row l % 16 of A and column l % 16 of B, eight consecutive
// k each (the same k for both), and rows 4 (l / 16) .. + 3 of column l % 16 of C.
#include "common.h"

namespace {

typedef _Float16 mm_half8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float mm_f16(uint16_t b) { return (float) __builtin_bit_cast(_Float16, b); }

// The matrix of a launch that row tile x falls in (segments in order), and x's tile within it.
struct MmSegView {
    const uint8_t *w;
    const float *bias;
    float *y;
    uint64_t row_bytes, part_off;
    uint32_t rows, y_stride, tile;
};
__device__ __forceinline__ MmSegView mm_seg(const MatmulArgs &a, uint32_t x) {
    uint32_t s = 0;
    while (s + 1u < a.n_seg && x >= a.seg[s].tile_end) ++s;
    const MatmulSeg &g = a.seg[s];
    return MmSegView{g.w, g.bias, g.y, g.row_bytes, g.part_off, g.rows, g.y_stride,
                     x - (s ? a.seg[s - 1u].tile_end : 0u)};
}

template <uint32_t TY, int RT, int NST>
__device__ __forceinline__ void matmul_body(const MatmulArgs &a) {
    // The work-group's activation tile of one k-block (64 tokens x 32 k, hi and lo) is staged in
    // LDS once and read by all four waves: fragment (quarter q, token t) at 16-byte slot q*64 + t,
    // so the 64 lanes of a fragment read touch 64 consecutive slots. Two buffers; one barrier per
    // k-block. Each thread copies the quarter tid/64 of token tid%64, hi and lo.
    __shared__ u32x4_t bsm[2][2][256];
    __shared__ float xsm[2][64];  // K-quants: the tile's per-token block sums
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t lr = lane & 15u, lq = lane >> 4;
    const MmSegView sg = mm_seg(a, blockIdx.x);
    const uint32_t r0 = sg.tile * (64u * RT) + 16u * RT * wave;  // RT 16-row tiles per wave
    const uint32_t t0 = blockIdx.y * MOEARC_MM_TOKENS;
    // this work-group's k-slice: blocks kb0 .. kb0 + nb (for the K-quants kb_per is a multiple of
    // 8, so the sub-block index b & 7 is the same counted from the slice or from the row's start)
    const uint32_t nb_all = a.cols / 32u, kb0 = blockIdx.z * a.kb_per;
    const uint32_t nb = min(a.kb_per, nb_all - kb0);
    const uint64_t kbyte0 = (uint64_t) kb0 * 32u / moearc_mv_be(TY) * moearc_mv_bb(TY);
    const uint8_t *wa[RT];  // this lane's A row (clamped: waves past the last row still stage)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
        wa[rt] = sg.w + (uint64_t) min(r0 + 16u * rt + lr, sg.rows - 1u) * sg.row_bytes + kbyte0;
    const uint64_t ct = min(t0 + (tid & 63u), a.n_tok - 1u);
    const uint16_t *cxh = a.xh + ct * a.cols + 32u * kb0 + 8u * (tid >> 6);
    const uint16_t *cxl = a.xl + ct * a.cols + 32u * kb0 + 8u * (tid >> 6);
    float4_t acc[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rt][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    struct Ops {  // raw loaded words, converted only when used, so a load never waits early
        uint16_t a[RT][8];   // Q8_0 / Q4_K / Q5_K payload words, F16 halves
        uint16_t h[RT][4];   // Q5_K fifth bits
        uint16_t d[RT][2];   // Q8_0 d; K-quant d, dmin
        uint8_t sc[RT][3];   // K-quant scale bytes of the sub-block
        uint32_t mx[RT][3];  // MXFP4: the aligned dwords around this lane's 8 payload bytes
        uint8_t e[RT];       // MXFP4 exponent
        u32x4_t xh, xl;      // this thread's share of the next activation tile
        float xsum;          // threads 0..63: the block sum of token tid
    };
    auto load = [&](uint32_t b, Ops &o) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if constexpr (TY == 8) {  // Q8_0: 34-byte blocks, f16 d then 32 int8
                const uint16_t *q = (const uint16_t *) (wa[rt] + 34u * b + 2u + 8u * lq);
#pragma unroll
                for (int i = 0; i < 4; ++i) o.a[rt][i] = q[i];
                o.d[rt][0] = *(const uint16_t *) (wa[rt] + 34u * b);
            } else if constexpr (TY == 1) {  // F16
                const uint16_t *h = (const uint16_t *) (wa[rt] + 2u * (32u * b + 8u * lq));
#pragma unroll
                for (int i = 0; i < 8; ++i) o.a[rt][i] = h[i];
            } else if constexpr (TY == 12 || TY == 13) {  // K-quants: sub-block s of super-block b / 8
                const uint32_t s = b & 7u;
                const uint8_t *sb = wa[rt] + (TY == 12 ? 144u : 176u) * (b >> 3);
                const uint16_t *q = (const uint16_t *) (sb + (TY == 12 ? 16u : 48u) + 32u * (s >> 1) + 8u * lq);
#pragma unroll
                for (int i = 0; i < 4; ++i) o.a[rt][i] = q[i];
                if constexpr (TY == 13) {
                    const uint16_t *qh = (const uint16_t *) (sb + 16u + 8u * lq);
#pragma unroll
                    for (int i = 0; i < 4; ++i) o.h[rt][i] = qh[i];
                }
                o.d[rt][0] = *(const uint16_t *) sb;
                o.d[rt][1] = *(const uint16_t *) (sb + 2u);
                o.sc[rt][0] = sb[4u + (s & 3u)];
                o.sc[rt][1] = sb[8u + (s & 3u)];
                o.sc[rt][2] = sb[12u + (s & 3u)];
            } else if constexpr (TY == 14) {  // Q6_K: k-block s = (half n, quarter c) of super-block b / 8
                const uint32_t s = b & 7u, n = s >> 2, c = s & 3u;
                const uint8_t *sb = wa[rt] + 210u * (b >> 3);
                const uint16_t *ql = (const uint16_t *) (sb + 64u * n + 32u * (c & 1u) + 8u * lq);
                const uint16_t *qh = (const uint16_t *) (sb + 128u + 32u * n + 8u * lq);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    o.a[rt][i] = ql[i];
                    o.h[rt][i] = qh[i];
                }
                o.d[rt][0] = *(const uint16_t *) (sb + 208u);
                o.sc[rt][0] = sb[192u + 8u * n + 2u * c];
                o.sc[rt][1] = sb[192u + 8u * n + 2u * c + 1u];
            } else {  // MXFP4: 17-byte blocks, E8M0 exponent then 16 bytes of nibble pairs
                const uint8_t *blk = wa[rt] + 17u * b;
                const uintptr_t at = (uintptr_t) (blk + 1u + 8u * (lq & 1u));
                const uint32_t *w4 = (const uint32_t *) (at & ~(uintptr_t) 3);
                o.mx[rt][0] = w4[0];
                o.mx[rt][1] = w4[1];
                // the third dword only holds wanted bytes when the eight are unaligned; otherwise
                // it could lie past the matrix, so the second is read again
                o.mx[rt][2] = w4[(at & 3u) ? 2 : 1];
                o.e[rt] = blk[0];
            }
        }
        o.xh = *(const u32x4_t *) (cxh + 32u * b);
        o.xl = *(const u32x4_t *) (cxl + 32u * b);
        if constexpr (TY == 12 || TY == 13)
            o.xsum = a.xs[ct * nb_all + kb0 + b];
    };
    auto stage = [&](const Ops &o, uint32_t buf) {
        bsm[buf][0][(tid >> 6) * 64u + (tid & 63u)] = o.xh;
        bsm[buf][1][(tid >> 6) * 64u + (tid & 63u)] = o.xl;
        if constexpr (TY == 12 || TY == 13)
            if (tid < 64u) xsm[buf][tid] = o.xsum;
    };
    auto operand_a = [&](const Ops &o, int rt, uint32_t b) {
        mm_half8 A;
        if constexpr (TY == 8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                A[2 * i] = (_Float16) (int8_t) (o.a[rt][i] & 0xFFu);
                A[2 * i + 1] = (_Float16) (int8_t) (o.a[rt][i] >> 8);
            }
        } else if constexpr (TY == 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i) A[i] = __builtin_bit_cast(_Float16, o.a[rt][i]);
        } else if constexpr (TY == 12 || TY == 13) {  // nibble (+ fifth bit), exact small integers
            const uint32_t s = b & 7u, sh = 4u * (s & 1u);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    uint32_t q = ((uint32_t) (o.a[rt][i] >> (8 * half)) >> sh) & 0xFu;
                    if constexpr (TY == 13) q |= (((uint32_t) (o.h[rt][i] >> (8 * half)) >> s) & 1u) << 4;
                    A[2 * i + half] = (_Float16) (uint16_t) q;
                }
            }
        } else if constexpr (TY == 14) {  // q - 32 in [-32, 31], exact
            const uint32_t c = (b & 7u) & 3u, shl = 4u * (c >> 1), shh = 2u * c;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const uint32_t lo = ((uint32_t) (o.a[rt][i] >> (8 * half)) >> shl) & 0xFu;
                    const uint32_t hi = ((uint32_t) (o.h[rt][i] >> (8 * half)) >> shh) & 3u;
                    A[2 * i + half] = (_Float16) ((int) (lo | (hi << 4)) - 32);
                }
            }
        } else {  // MXFP4: E2M1 code points as f16 bits (exact)
            const uintptr_t at = (uintptr_t) (wa[rt] + 17u * b + 1u + 8u * (lq & 1u));
            const uint32_t sh = (uint32_t) (at & 3u);
            const uint32_t lo = __builtin_amdgcn_alignbyte(o.mx[rt][1], o.mx[rt][0], sh);
            const uint32_t hi = __builtin_amdgcn_alignbyte(o.mx[rt][2], o.mx[rt][1], sh);
            const uint32_t nsh = 4u * (lq >> 1);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t byte = ((i < 4 ? lo : hi) >> (8 * (i & 3))) & 0xFFu;
                const uint32_t c = (byte >> nsh) & 0xFu, mag = c & 7u;
                const uint32_t bits = mag == 0u ? 0u : mag == 1u ? 0x3800u : (((mag >> 1) + 14u) << 10) | ((mag & 1u) << 9);
                A[i] = __builtin_bit_cast(_Float16, (uint16_t) (bits | ((c & 8u) << 12)));
            }
        }
        return A;
    };
    // Per-row scale (and min) of this lane's A row for k-block b; moved to the accumulator rows
    // 4 lq + k with ds_bpermute.
    auto row_scales = [&](const Ops &o, int rt, uint32_t b, float &sc1, float &mn1) {
        if constexpr (TY == 8) {
            sc1 = mm_f16(o.d[rt][0]);
            mn1 = 0.f;
        } else if constexpr (TY == 12 || TY == 13) {
            const uint32_t s = b & 7u;
            const uint32_t r0b = o.sc[rt][0], r1b = o.sc[rt][1], r2b = o.sc[rt][2];
            const bool low = s < 4u;  // get_scale_min_k4 (reference.rs:150-160)
            const uint32_t sc = low ? (r0b & 63u) : ((r2b & 0xFu) | ((r0b >> 6) << 4));
            const uint32_t m = low ? (r1b & 63u) : ((r2b >> 4) | ((r1b >> 6) << 4));
            sc1 = mm_f16(o.d[rt][0]) * (float) sc;
            mn1 = mm_f16(o.d[rt][1]) * (float) m;
        } else if constexpr (TY == 14) {  // the two 16-wide groups' d * sc
            const float d = mm_f16(o.d[rt][0]);
            sc1 = d * (float) (int8_t) o.sc[rt][0];
            mn1 = d * (float) (int8_t) o.sc[rt][1];
        } else {  // MXFP4: 2^(e - 127)
            sc1 = __uint_as_float(o.e[rt] ? (uint32_t) o.e[rt] << 23 : 0x00400000u);
            mn1 = 0.f;
        }
    };
    auto compute = [&](const Ops &o, uint32_t buf, uint32_t b) {
        mm_half8 bh[4], bl[4];
        float xsv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bh[j] = __builtin_bit_cast(mm_half8, bsm[buf][0][lq * 64u + 16u * j + lr]);
            bl[j] = __builtin_bit_cast(mm_half8, bsm[buf][1][lq * 64u + 16u * j + lr]);
            if constexpr (TY == 12 || TY == 13) xsv[j] = xsm[buf][16u * j + lr];
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const mm_half8 A = operand_a(o, rt, b);
            float dk[4], mk[4];
            if constexpr (TY != 1) {
                float sc1, mn1;
                row_scales(o, rt, b, sc1, mn1);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int src = (int) ((4u * lq + k) << 2);
                    dk[k] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(sc1)));
                    if constexpr (TY == 12 || TY == 13 || TY == 14)
                        mk[k] = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(mn1)));
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (TY == 1) {
                    acc[rt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bh[j], acc[rt][j], 0, 0, 0);
                    acc[rt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bl[j], acc[rt][j], 0, 0, 0);
                } else if constexpr (TY == 14) {
                    // two 16-wide scale groups in one k-block: lanes 0-31 hold group 0's k, 32-63
                    // group 1's, so each group's sum is an MFMA with the other group's A zeroed
                    float4_t sg[2];
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        const mm_half8 Ag = (lq >> 1) == (uint32_t) g ? A : mm_half8{};
                        sg[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ag, bh[j], float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        sg[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ag, bl[j], sg[g], 0, 0, 0);
                    }
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        acc[rt][j][k] = fmaf(mk[k], sg[1][k], fmaf(dk[k], sg[0][k], acc[rt][j][k]));
                } else {
                    float4_t s = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bh[j], float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bl[j], s, 0, 0, 0);
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        acc[rt][j][k] = fmaf(dk[k], s[k], acc[rt][j][k]);
                        if constexpr (TY == 12 || TY == 13) acc[rt][j][k] = fmaf(-mk[k], xsv[j], acc[rt][j][k]);
                    }
                }
            }
        }
    };
    // NST operand sets in flight: k-block k lives in set k % NST, and block b + NST - 1 is
    // requested (clamped at the end, so every step issues the same loads) before block b's
    // products. Block b + 1's activation share reaches LDS after block b's products, then the
    // work-group meets once (two LDS buffers: a buffer is refilled only after every wave has
    // passed the barrier that follows the products that read it).
    Ops ops[NST];
#pragma unroll
    for (int s = 0; s < NST - 1; ++s) load(min((uint32_t) s, nb - 1u), ops[s]);
    stage(ops[0], 0);
    __syncthreads();
    uint32_t b = 0;
    for (; b + NST <= nb; b += NST) {
#pragma unroll
        for (int s = 0; s < NST; ++s) {
            load(min(b + (uint32_t) (s + NST - 1), nb - 1u), ops[(s + NST - 1) % NST]);
            __builtin_amdgcn_sched_barrier(0);
            compute(ops[s], (b + s) & 1u, b + s);
            stage(ops[(s + 1) % NST], (b + s + 1u) & 1u);
            __syncthreads();
        }
    }
#pragma unroll
    for (int s = 0; s < NST; ++s) {
        if (b + s < nb) {
            compute(ops[s], (b + s) & 1u, b + s);
            if (b + s + 1u < nb) {
                stage(ops[(s + 1) % NST], (b + s + 1u) & 1u);
                __syncthreads();
            }
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t t = t0 + 16u * j + lr;
            if (t >= a.n_tok) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t r = r0 + 16u * rt + 4u * lq + k;
                if (r < sg.rows) {
                    if (gridDim.z > 1) {  // one slice of a split launch: its sums, for the reduction
                        a.part[blockIdx.z * a.part_stride + sg.part_off + (uint64_t) t * sg.rows + r] = acc[rt][j][k];
                        continue;
                    }
                    float *yp = sg.y + (uint64_t) t * sg.y_stride + r;
                    const float v = sg.bias ? acc[rt][j][k] + sg.bias[r] : acc[rt][j][k];
                    *yp = a.accumulate ? *yp + v : v;
                }
            }
        }
}

}  // namespace

#ifndef MM_STAGES
#define MM_STAGES 2  // k-blocks of operands in flight per wave
#endif

// _r1: 16 rows per wave (more work-groups, for short chunks); _r2: 32 rows per wave.
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q4_k_r1_k(MatmulArgs a) { matmul_body<12, 1, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q4_k_r2_k(MatmulArgs a) { matmul_body<12, 2, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q5_k_r1_k(MatmulArgs a) { matmul_body<13, 1, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q5_k_r2_k(MatmulArgs a) { matmul_body<13, 2, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q6_k_r1_k(MatmulArgs a) { matmul_body<14, 1, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q6_k_r2_k(MatmulArgs a) { matmul_body<14, 2, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_mxfp4_r1_k(MatmulArgs a) { matmul_body<39, 1, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_mxfp4_r2_k(MatmulArgs a) { matmul_body<39, 2, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q8_0_r1_k(MatmulArgs a) { matmul_body<8, 1, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q8_0_r2_k(MatmulArgs a) { matmul_body<8, 2, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_f16_r1_k(MatmulArgs a) { matmul_body<1, 1, MM_STAGES>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_f16_r2_k(MatmulArgs a) { matmul_body<1, 2, MM_STAGES>(a); }

// x -> (hi, lo) f16 with hi = f16(x), lo = f16(x - hi), both round-to-nearest-even.
extern "C" __global__ void moearc_split_f16_k(const float *x, uint16_t *hi, uint16_t *lo, uint64_t n) {
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t) gridDim.x * blockDim.x) {
        const float v = x[i];
        const _Float16 h = (_Float16) v;
        const _Float16 l = (_Float16) (v - (float) h);
        hi[i] = __builtin_bit_cast(uint16_t, h);
        lo[i] = __builtin_bit_cast(uint16_t, l);
    }
}

// moearc_split_f16_k eight elements at a time (x 16-byte aligned, n a multiple of 8): two 16-byte
// loads and two 16-byte stores per thread instead of one element and two 2-byte stores, the stores
// written through to the device-coherent level (whole lines per wave, so the kernel's end has no
// dirty L2 lines of the two halves to write back). Same arithmetic, same results.
extern "C" __global__ void moearc_split_f16_v8_k(const float *x, uint16_t *hi, uint16_t *lo, uint64_t n8) {
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n8;
         i += (uint64_t) gridDim.x * blockDim.x) {
        const float4_t va = ((const float4_t *) x)[2 * i], vb = ((const float4_t *) x)[2 * i + 1];
        half8_t h, l;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            h[k] = (_Float16) va[k];
            l[k] = (_Float16) (va[k] - (float) h[k]);
            h[4 + k] = (_Float16) vb[k];
            l[4 + k] = (_Float16) (vb[k] - (float) h[4 + k]);
        }
        store_through16((u32x4_t *) hi + i, __builtin_bit_cast(u32x4_t, h));
        store_through16((u32x4_t *) lo + i, __builtin_bit_cast(u32x4_t, l));
    }
}

// xs[i] = the sum of x[32 i .. 32 i + 31], in order, in f32: the per-(token, k-block) activation
// sums of the K-quant chunk products.
extern "C" __global__ void moearc_block_sums_k(const float *x, float *xs, uint64_t n_blocks) {
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n_blocks;
         i += (uint64_t) gridDim.x * blockDim.x) {
        const float *p = x + 32u * i;
        float t = 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j) t += p[j];
        xs[i] = t;
    }
}

// The reduction of a split launch: y[t][r] = the sum of the n_slices k-slices' sums (in slice
// order) + bias[r], added to y[t][r] when a.accumulate -- the single launch's epilogue with the
// sum taken over slices -- for every matrix of the launch.
extern "C" __global__ void moearc_matmul_reduce_k(MatmulArgs a, uint32_t n_slices) {
    const uint64_t n = a.part_stride;
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t) gridDim.x * blockDim.x) {
        // this element's matrix, chosen by selects between the (uniform) segment fields: indexing
        // the argument block with a per-lane value would cost a memory round trip first
        const bool s1 = a.n_seg > 1u && i >= a.seg[1].part_off, s2 = a.n_seg > 2u && i >= a.seg[2].part_off;
        auto pick = [&](auto f0, auto f1, auto f2) { return s2 ? f2 : s1 ? f1 : f0; };
        const uint64_t part_off = pick(a.seg[0].part_off, a.seg[1].part_off, a.seg[2].part_off);
        const uint32_t rows = pick(a.seg[0].rows, a.seg[1].rows, a.seg[2].rows);
        const uint32_t y_stride = pick(a.seg[0].y_stride, a.seg[1].y_stride, a.seg[2].y_stride);
        float *const y = pick(a.seg[0].y, a.seg[1].y, a.seg[2].y);
        const float *const bias = pick(a.seg[0].bias, a.seg[1].bias, a.seg[2].bias);
        const uint64_t e = i - part_off;
        const uint32_t t = (uint32_t) (e / rows), r = (uint32_t) (e - (uint64_t) t * rows);
        float *yp = y + (uint64_t) t * y_stride + r;
        // the residual (when accumulating), the bias and eight slices' loads in flight at a time, added in
        // slice order; a last group short of eight reads slice n_slices - 1 in the missing places
        // and leaves those values out, so that every group's loads leave before its first add
        const float prev = a.accumulate ? *yp : 0.f;
        const float bv = bias ? bias[r] : 0.f;
        float s = 0.f;
        for (uint32_t z = 0; z < n_slices; z += 8u) {
            float v[8];
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k) v[k] = a.part[(uint64_t) min(z + k, n_slices - 1u) * n + i];
#pragma unroll
            for (uint32_t k = 0; k < 8u; ++k)
                s = z + k == 0u ? v[k] : z + k < n_slices ? s + v[k] : s;
        }
        const float v = bias ? s + bv : s;
        *yp = a.accumulate ? prev + v : v;
    }
}

// The same, four consecutive elements of a row per lane (every matrix's rows, y_stride and
// part_off, the part stride and the y, bias and part addresses multiples of 4 floats, checked by
// the host) and up to 16 slices' loads in flight before the first add: one round trip for the
// slice counts the host picks. Per element the additions and their order are the scalar kernel's.
extern "C" __global__ void moearc_matmul_reduce4_k(MatmulArgs a, uint32_t n_slices) {
    const uint64_t n = a.part_stride;
    for (uint64_t i = 4u * ((uint64_t) blockIdx.x * blockDim.x + threadIdx.x); i < n;
         i += 4u * (uint64_t) gridDim.x * blockDim.x) {
        const bool s1 = a.n_seg > 1u && i >= a.seg[1].part_off, s2 = a.n_seg > 2u && i >= a.seg[2].part_off;
        auto pick = [&](auto f0, auto f1, auto f2) { return s2 ? f2 : s1 ? f1 : f0; };
        const uint64_t part_off = pick(a.seg[0].part_off, a.seg[1].part_off, a.seg[2].part_off);
        const uint32_t rows = pick(a.seg[0].rows, a.seg[1].rows, a.seg[2].rows);
        const uint32_t y_stride = pick(a.seg[0].y_stride, a.seg[1].y_stride, a.seg[2].y_stride);
        float *const y = pick(a.seg[0].y, a.seg[1].y, a.seg[2].y);
        const float *const bias = pick(a.seg[0].bias, a.seg[1].bias, a.seg[2].bias);
        const uint64_t e = i - part_off;
        const uint32_t t = (uint32_t) (e / rows), r = (uint32_t) (e - (uint64_t) t * rows);
        float4_t *yp = (float4_t *) (y + (uint64_t) t * y_stride + r);
        const float4_t prev = a.accumulate ? *yp : float4_t{0.f, 0.f, 0.f, 0.f};
        const float4_t bv = bias ? *(const float4_t *) (bias + r) : float4_t{0.f, 0.f, 0.f, 0.f};
        float4_t s = {0.f, 0.f, 0.f, 0.f};
        for (uint32_t z = 0; z < n_slices; z += 16u) {
            float4_t v[16];
#pragma unroll
            for (uint32_t k = 0; k < 16u; ++k)
                v[k] = *(const float4_t *) (a.part + (uint64_t) min(z + k, n_slices - 1u) * n + i);
#pragma unroll
            for (uint32_t k = 0; k < 16u; ++k)
                s = z + k == 0u ? v[k] : z + k < n_slices ? s + v[k] : s;
        }
        const float4_t v = bias ? s + bv : s;
        *yp = a.accumulate ? prev + v : v;
    }
}
