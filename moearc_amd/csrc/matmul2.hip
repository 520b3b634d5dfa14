// Chunk-form projections for Q8_0 and F16 weights on v_mfma_f32_32x32x16_f16:
// Y[t][r] = sum_c W[r][c] X[t][c] (+ bias[r]) for the tokens of a prompt chunk -- the GEMM that the
// reference's prefill performs as one matvec per token (moe.rs:1942-1959, 2063-2071;
// kernels.cpp:1046-1111). Precision is matmul.hip's: X is split into f16 hi + lo on the host side of
// the launch (x - hi - lo <= 2^-22 |x|), a Q8_0 block's payload enters the MFMA as exact f16
// integers, each 32-wide block's f32 sum q . (hi + lo) is scaled by the block's d in f32; F16
// weights enter as they are. Activations must stay below 65504 in magnitude.
//
// The product is computed transposed, D[token][row] = X . W^T, so that the weight rows are the MFMA's
// N side: lane l holds D column l % 32 -- one weight row -- in all 16 of its accumulators, and a
// Q8_0 block scale is one per-lane multiplier (it is also the lane that loaded that row's block).
// Within a 32-wide k-block, lane (n, h) (h = l >> 5) feeds k 16h + 8s .. + 7 to the MFMA of k
// slice s, for both operands: its weight bytes for the block are then one contiguous 16-byte
// piece (a single load per row tile; the weight loads touch one cache line per row and lane pair
// per instruction, and the fewer such instructions per step, the faster the step).
//
// Work-group: 4 waves over 128 tokens x 128 weight rows; wave w takes tokens 64 (w & 1) .. + 63 and
// rows 64 (w >> 1) .. + 63 as 2 x 2 tiles of 32 x 32. Per 32-wide k-block the work-group's
// activation tile (128 tokens x 32 k, hi and lo: 16 KiB) arrives in LDS by LDS DMA
// (global_load_lds_dwordx4, 16 bytes per lane at the wave's base + 16 lane), three buffers, two
// k-blocks ahead; each wave loads its own weight rows into registers, also two k-blocks ahead. One
// barrier per k-block. LDS layout per half: token t's 64-byte row holds 16-byte chunk c (k 8c..8c+7)
// at position c ^ swz(t), swz(t) = ((t >> 2) + 2 (t >> 4)) & 3, so that every 16-lane group of an
// operand read (tokens t..t+15, or t..t+7 and t+16..t+23, one chunk) touches 64 distinct banks.
#include "common.h"

namespace {

constexpr uint32_t MM2_TOK = 128;   // tokens per work-group
constexpr uint32_t MM2_ROWS = 128;  // weight rows per work-group
constexpr uint32_t MM2_HALF = MM2_TOK * 64u;  // bytes of one half (hi or lo) of an activation tile
constexpr uint32_t MM2_BUF = 2u * MM2_HALF;   // one k-block's activation tile
constexpr uint32_t MM2_NBUF = 3u;
// fewest memory instructions one block's weight loads compile to (Q8_0: per row tile 16 int8 and
// the scale; F16: per row tile two 16-byte pieces of 8 halves)
constexpr uint32_t MM2_WLOADS = 4u;

typedef float mm2_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t mm2_u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t mm2_swz(uint32_t t) { return ((t >> 2) + ((t >> 4) << 1)) & 3u; }

// s_waitcnt immediates (gfx9 encoding): vmcnt <= n and nothing else; vmcnt <= n and lgkmcnt 0
constexpr uint32_t mm2_vmcnt(uint32_t n) { return (n & 0xFu) | ((n >> 4) << 14) | (0x7u << 4) | (0xFu << 8); }
constexpr uint32_t mm2_vmcnt_lgkm0(uint32_t n) { return (n & 0xFu) | ((n >> 4) << 14) | (0x7u << 4); }

// 8 int8 in two dwords -> 8 exact f16: (q ^ 0x80) in the low byte under exponent 0x64 is 1024 + q + 128
__device__ __forceinline__ half8_t mm2_i8_to_f16(mm2_u32x2 q) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t x = q[i] ^ 0x80808080u;
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
        const half2_t h0 = __builtin_bit_cast(half2_t, p0) - half2_t{(_Float16) 1152.f, (_Float16) 1152.f};
        const half2_t h1 = __builtin_bit_cast(half2_t, p1) - half2_t{(_Float16) 1152.f, (_Float16) 1152.f};
        r[4 * i] = h0[0];
        r[4 * i + 1] = h0[1];
        r[4 * i + 2] = h1[0];
        r[4 * i + 3] = h1[1];
    }
    return r;
}

template <uint32_t TY>
struct Mm2W;  // one k-block of this lane's weight operands, raw
template <>
struct Mm2W<8> {  // Q8_0: per row tile this lane's 16 int8 (k 16h .. 16h + 15); the block's d
    u32x4_t q[2];
    uint16_t d[2];
};
template <>
struct Mm2W<1> {  // F16: per row tile and k slice 8 halves
    u32x4_t h[2][2];
};

template <uint32_t TY>
__device__ __forceinline__ void mm2_body(const MatmulArgs &a) {
    __shared__ __attribute__((aligned(1024))) uint8_t tiles[MM2_NBUF * MM2_BUF];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 31u, h = lane >> 5;
    const MmSegView sg = mm_seg(a, blockIdx.x);
    const uint32_t t0 = blockIdx.y * MM2_TOK, r0 = sg.tile * MM2_ROWS;
    // this work-group's k-slice: blocks kb0 .. kb0 + nb
    const uint32_t kb0 = blockIdx.z * a.kb_per, nb = min(a.kb_per, a.cols / 32u - kb0);
    const uint32_t lds0 = (uint32_t) (uintptr_t) (__attribute__((address_space(3))) uint8_t *) tiles;

    // LDS DMA: instruction i of wave w fills region R = 4 w + i (1 KiB): half R >> 3, tokens
    // 16 (R & 7) .. + 15; lane L writes slot L of the region = chunk position L & 3 of token L >> 2,
    // which holds chunk (L & 3) ^ swz(token).
    const uint16_t *dma_src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t R = 4u * wave + (uint32_t) i;
        const uint32_t tok = 16u * (R & 7u) + (lane >> 2);
        const uint32_t c = (lane & 3u) ^ mm2_swz(tok);
        const uint64_t tg = min(t0 + tok, a.n_tok - 1u);
        dma_src[i] = ((R >> 3) ? a.xl : a.xh) + tg * a.cols + 32u * kb0 + 8u * c;
    }
    // The copies are issued as asm (m0 saved and restored, memory clobbered), out of the compiler's
    // wait bookkeeping: with LDS-DMA operations in flight it cannot count the weight loads' waits
    // and drains every memory operation (vmcnt(0)) before each step's MFMAs -- the requests just
    // made for two blocks ahead included. The step's leading wait covers the copies; the compiler
    // counts its own weight loads (copies issued between them only make its waits longer).
    auto dma = [&](uint32_t b, uint32_t buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t R = 4u * wave + (uint32_t) i;
            const uint32_t lds = __builtin_amdgcn_readfirstlane(lds0 + buf * MM2_BUF + R * 1024u);
            uint32_t m0_saved;
            asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                         "global_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                         : "=&s"(m0_saved)
                         : "s"(lds), "v"(dma_src[i] + 32u * b)
                         : "memory");
        }
    };

    // this lane's weight rows (clamped: lanes past the last row load row rows - 1 and store nothing)
    const uint8_t *wrow[2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
        wrow[rt] = sg.w + (uint64_t) min(r0 + 64u * (wave >> 1) + 32u * rt + n, sg.rows - 1u) * sg.row_bytes +
                   (TY == 8 ? 34u : 64u) * (uint64_t) kb0;
    auto wload = [&](uint32_t b, Mm2W<TY> &o) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            if constexpr (TY == 8) {
                const uint8_t *blk = wrow[rt] + 34u * b;
                o.d[rt] = *(const uint16_t *) blk;
                __builtin_memcpy(&o.q[rt], blk + 2u + 16u * h, 16);
            } else {
#pragma unroll
                for (int s = 0; s < 2; ++s)
                    o.h[rt][s] = *(const u32x4_t *) (wrow[rt] + 2u * (32u * b + 16u * h + 8u * s));
            }
        }
    };

    mm2_f32x16 acc[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[tt][rt][j] = 0.f;

    // A operand (activations) of token tile tt, k slice s: token 64 (w & 1) + 32 tt + n, chunk 2 h + s
    uint32_t aoff[2][2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const uint32_t tok = 64u * (wave & 1u) + 32u * tt + n;
            aoff[tt][s] = lds0 + tok * 64u + 16u * ((2u * h + s) ^ mm2_swz(tok));
        }
    auto compute = [&](uint32_t buf, const Mm2W<TY> &o) {
        half8_t ah[2][2], al[2][2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const uint32_t off = aoff[tt][s] + buf * MM2_BUF;
                ah[tt][s] = __builtin_bit_cast(half8_t, *(const __attribute__((address_space(3))) u32x4_t *) (uintptr_t) off);
                al[tt][s] = __builtin_bit_cast(half8_t,
                                               *(const __attribute__((address_space(3))) u32x4_t *) (uintptr_t) (off + MM2_HALF));
            }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            half8_t bw[2];
            if constexpr (TY == 8) {
#pragma unroll
                for (int s = 0; s < 2; ++s) bw[s] = mm2_i8_to_f16(mm2_u32x2{o.q[rt][2 * s], o.q[rt][2 * s + 1]});
            } else {
#pragma unroll
                for (int s = 0; s < 2; ++s) bw[s] = __builtin_bit_cast(half8_t, o.h[rt][s]);
            }
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                if constexpr (TY == 8) {
                    mm2_f32x16 sblk = {};
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        sblk = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tt][s], bw[s], sblk, 0, 0, 0);
                        sblk = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tt][s], bw[s], sblk, 0, 0, 0);
                    }
                    const float d = (float) __builtin_bit_cast(_Float16, o.d[rt]);
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[tt][rt][j] = fmaf(d, sblk[j], acc[tt][rt][j]);
                } else {
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        acc[tt][rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tt][s], bw[s], acc[tt][rt], 0, 0, 0);
                        acc[tt][rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tt][s], bw[s], acc[tt][rt], 0, 0, 0);
                    }
                }
            }
        }
    };

    // k-block b's activations in buffer b % 3, its weights in set b % 3. Step b: wait for block b's
    // DMA, meet the other waves (every wave has finished block b - 1, whose buffer is refilled
    // next), request block b + 2 (its DMA first, then its weights), compute block b. Issued after
    // block b's DMA are its weights and block b + 1's DMA and weights: at least 2 MM2_WLOADS + 4
    // memory operations (the weight loads of one block are at least MM2_WLOADS instructions), so
    // waiting until that many remain leaves both blocks' requests in flight.
    Mm2W<TY> ws[3];
    dma(0, 0);
    wload(0, ws[0]);
    dma(min(1u, nb - 1u), 1);
    wload(min(1u, nb - 1u), ws[1]);
    auto step = [&](uint32_t b, int s) {
        // block b's DMA has landed and every LDS read of block b - 1 has returned, in this wave;
        // then in every wave
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(mm2_vmcnt_lgkm0(2u * MM2_WLOADS + 4u));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t bn = min(b + 2u, nb - 1u);
        dma(bn, (uint32_t) (s + 2) % 3u);
        wload(bn, ws[(s + 2) % 3]);
        __builtin_amdgcn_sched_barrier(0);
        compute((uint32_t) s, ws[s]);
    };
    uint32_t b = 0;
    for (; b + 3u <= nb; b += 3u) {
        step(b, 0);
        step(b + 1u, 1);
        step(b + 2u, 2);
    }
    if (b < nb) step(b, 0);
    if (b + 1u < nb) step(b + 1u, 1);
    __builtin_amdgcn_s_waitcnt(mm2_vmcnt(0));  // no DMA outlives the work-group

    // D[token][row]: lane l holds row r0 + 64 (w >> 1) + 32 rt + n, tokens 8 (j / 4) + 4 h + j % 4 of
    // tile tt -- 32 consecutive rows per store instruction
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const uint32_t r = r0 + 64u * (wave >> 1) + 32u * rt + n;
        if (r >= sg.rows) continue;
        if (gridDim.z > 1) {  // one slice of a split launch: its sums, for the reduction
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const uint32_t t = t0 + 64u * (wave & 1u) + 32u * tt + 8u * (j >> 2) + 4u * h + (j & 3);
                    if (t < a.n_tok)
                        a.part[blockIdx.z * a.part_stride + sg.part_off + (uint64_t) t * sg.rows + r] = acc[tt][rt][j];
                }
            continue;
        }
        const float bias = sg.bias ? sg.bias[r] : 0.f;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t t = t0 + 64u * (wave & 1u) + 32u * tt + 8u * (j >> 2) + 4u * h + (j & 3);
                if (t < a.n_tok) {
                    float *yp = sg.y + (uint64_t) t * sg.y_stride + r;
                    const float v = acc[tt][rt][j] + bias;
                    *yp = a.accumulate ? *yp + v : v;
                }
            }
    }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256) moearc_matmul2_q8_0_k(MatmulArgs a) { mm2_body<8>(a); }
extern "C" __global__ void __launch_bounds__(256) moearc_matmul2_f16_k(MatmulArgs a) { mm2_body<1>(a); }
