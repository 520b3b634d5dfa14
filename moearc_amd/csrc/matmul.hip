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

template <uint32_t TY, int RT>
__device__ __forceinline__ void matmul_body(const MatmulArgs &a) {
    // The work-group's activation tile of one k-block (64 tokens x 32 k, hi and lo) is staged in
    // LDS once and read by all four waves: fragment (quarter q, token t) at 16-byte slot q*64 + t,
    // so the 64 lanes of a fragment read touch 64 consecutive slots. Two buffers; one barrier per
    // k-block. Each thread copies the quarter tid/64 of token tid%64, hi and lo.
    __shared__ u32x4_t bsm[2][2][256];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t lr = lane & 15u, lq = lane >> 4;
    const uint32_t r0 = blockIdx.x * (64u * RT) + 16u * RT * wave;  // RT 16-row tiles per wave
    const uint32_t t0 = blockIdx.y * MOEARC_MM_TOKENS;
    const uint32_t nb = a.cols / 32u;
    const uint8_t *wa[RT];  // this lane's A row (clamped: waves past the last row still stage)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) wa[rt] = a.w + (uint64_t) min(r0 + 16u * rt + lr, a.rows - 1u) * a.row_bytes;
    const uint64_t ct = min(t0 + (tid & 63u), a.n_tok - 1u);
    const uint16_t *cxh = a.xh + ct * a.cols + 8u * (tid >> 6);
    const uint16_t *cxl = a.xl + ct * a.cols + 8u * (tid >> 6);
    float4_t acc[RT][4];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[rt][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    struct Ops {  // raw loaded words, converted only when used, so a load never waits early
        uint16_t a[RT][8];
        uint16_t d[RT];      // the block scale of this lane's A row
        u32x4_t xh, xl;      // this thread's share of the next activation tile
    };
    auto load = [&](uint32_t b, Ops &o) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            if constexpr (TY == 8) {  // Q8_0: 34-byte blocks, f16 d then 32 int8
                const uint16_t *q = (const uint16_t *) (wa[rt] + 34u * b + 2u + 8u * lq);
#pragma unroll
                for (int i = 0; i < 4; ++i) o.a[rt][i] = q[i];
                o.d[rt] = *(const uint16_t *) (wa[rt] + 34u * b);
            } else {  // F16
                const uint16_t *h = (const uint16_t *) (wa[rt] + 2u * (32u * b + 8u * lq));
#pragma unroll
                for (int i = 0; i < 8; ++i) o.a[rt][i] = h[i];
            }
        }
        o.xh = *(const u32x4_t *) (cxh + 32u * b);
        o.xl = *(const u32x4_t *) (cxl + 32u * b);
    };
    auto stage = [&](const Ops &o, uint32_t buf) {
        bsm[buf][0][(tid >> 6) * 64u + (tid & 63u)] = o.xh;
        bsm[buf][1][(tid >> 6) * 64u + (tid & 63u)] = o.xl;
    };
    auto operand_a = [&](const Ops &o, int rt) {
        mm_half8 A;
        if constexpr (TY == 8) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                A[2 * i] = (_Float16) (int8_t) (o.a[rt][i] & 0xFFu);
                A[2 * i + 1] = (_Float16) (int8_t) (o.a[rt][i] >> 8);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) A[i] = __builtin_bit_cast(_Float16, o.a[rt][i]);
        }
        return A;
    };
    auto compute = [&](const Ops &o, uint32_t buf) {
        mm_half8 bh[4], bl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bh[j] = __builtin_bit_cast(mm_half8, bsm[buf][0][lq * 64u + 16u * j + lr]);
            bl[j] = __builtin_bit_cast(mm_half8, bsm[buf][1][lq * 64u + 16u * j + lr]);
        }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const mm_half8 A = operand_a(o, rt);
            float dk[4];
            if constexpr (TY == 8) {  // scales of accumulator rows 4 lq + k, from the lanes holding them
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    dk[k] = mm_f16((uint16_t) __builtin_amdgcn_ds_bpermute((int) ((4u * lq + k) << 2), (int) o.d[rt]));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (TY == 8) {
                    float4_t s = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bh[j], float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bl[j], s, 0, 0, 0);
#pragma unroll
                    for (int k = 0; k < 4; ++k) acc[rt][j][k] = fmaf(dk[k], s[k], acc[rt][j][k]);
                } else {
                    acc[rt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bh[j], acc[rt][j], 0, 0, 0);
                    acc[rt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, bl[j], acc[rt][j], 0, 0, 0);
                }
            }
        }
    };
    // Ping-pong: block b + 1's operands are requested (clamped at the end, so every iteration
    // issues the same loads) before block b's products; they reach LDS after them, then the
    // work-group meets once.
    Ops p, q;
    load(0, p);
    stage(p, 0);
    __syncthreads();
    uint32_t b = 0;
    for (; b + 1u < nb; b += 2u) {
        load(b + 1u, q);
        __builtin_amdgcn_sched_barrier(0);
        compute(p, 0);
        stage(q, 1);
        __syncthreads();
        load(min(b + 2u, nb - 1u), p);
        __builtin_amdgcn_sched_barrier(0);
        compute(q, 1);
        stage(p, 0);
        __syncthreads();
    }
    if (b < nb) compute(p, 0);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t t = t0 + 16u * j + lr;
            if (t >= a.n_tok) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t r = r0 + 16u * rt + 4u * lq + k;
                if (r < a.rows)
                    a.y[(uint64_t) t * a.y_stride + r] = a.bias ? acc[rt][j][k] + a.bias[r] : acc[rt][j][k];
            }
        }
}

}  // namespace

// _r1: 16 rows per wave (more work-groups, for short chunks); _r2: 32 rows per wave.
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q8_0_r1_k(MatmulArgs a) { matmul_body<8, 1>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_q8_0_r2_k(MatmulArgs a) { matmul_body<8, 2>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_f16_r1_k(MatmulArgs a) { matmul_body<1, 1>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul_f16_r2_k(MatmulArgs a) { matmul_body<1, 2>(a); }

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
