// Chunk-form projections on v_mfma_f32_32x32x16_f16, for F16, Q8_0, Q4_K, Q5_K, Q6_K and MXFP4
// weights: Y[t][r] = sum_c W[r][c] X[t][c] (+ bias[r]) for the tokens of a prompt chunk -- the GEMM
// that the reference's prefill performs as one matvec per token (moe.rs:1942-1959, 2063-2071;
// kernels.cpp:1046-1111). Precision is matmul.hip's: X is split into f16 hi + lo on the host side of
// the launch (x - hi - lo <= 2^-22 |x|), a block's payload enters the MFMA as exact f16 integers
// (E2M1 code points for MXFP4), each 32-wide block's (Q6_K: 16-wide group's) f32 sum q . (hi + lo)
// is scaled by the block's factor in f32 (and, for Q4_K and Q5_K, its min times the activation's
// block sum subtracted); F16 weights enter as they are. Activations must stay below 65504.
//
// The product is computed transposed, D[token][row] = X . W^T, so that the weight rows are the MFMA's
// N side: lane l holds D column l % 32 -- one weight row -- in all 16 of its accumulators, and a
// Q8_0 block scale is one per-lane multiplier. Within a 32-wide k-block, lane (n, h) (h = l >> 5)
// feeds k 16h + 8s .. + 7 to the MFMA of k slice s, for both operands.
//
// Work-group: 4 waves over 128 tokens x 128 weight rows; wave w takes tokens 64 (w & 1) .. + 63 and
// rows 64 (w >> 1) .. + 63 as 2 x 2 tiles of 32 x 32. F16, Q8_0 and MXFP4 also come as a wide form, 8
// waves over 128 tokens x 256 rows, one work-group per CU: the same waves' steps, with each
// k-block's copies shared by twice the rows (the CU's intake of copied bytes costs time beside
// the MFMAs, whatever the copies' destination). Both operands reach LDS by LDS DMA
// (global_load_lds_dwordx4: 16 bytes per lane, written at the instruction's LDS base + 16 lane),
// two k-blocks ahead, and are read from there in operand layout; one barrier per k-block. Every
// copy reads 64-byte row pieces, four lanes per row: a memory instruction costs in proportion to
// the cache lines it touches, and loading weights straight into operand layout touches one line
// per row for 16 useful bytes (measured: that form spends a third of the product's time there).
// - Activations: per k-block 128 tokens x 32 k, hi and lo (16 KiB); three buffers. Token t's
//   64-byte row holds 16-byte chunk c (k 8c .. 8c + 7) at position c ^ swz(t), swz(t) = (t >> 2)
//   & 3: the 16-byte operand reads then measure free of bank conflicts (SQ_LDS_BANK_CONFLICT 0 in
//   the F16 kernel; 4 cycles per read with 2 (t >> 4) added to swz, 12 with no swizzle).
// - F16 weights: per k-block 128 rows x 64 bytes in the same layout, beside each activation tile.
// - Q8_0 weights, per pair of k-blocks: a row's 68 bytes (d0, q0[32], d1, q1[32]) as four 16-byte
//   chunks (bytes 0 .. 63, same layout) plus a 4-byte tail array (bytes 64 .. 67); three pair
//   buffers. Lane (n, h) takes its 16 payload bytes of block 0 from chunk h and the first dword of
//   chunk h + 1 (window bytes 2 + 16h ..: one v_alignbyte per dword), those of block 1 from chunk
//   h + 2 and the first dword of chunk 3 or the tail (dword-aligned), and the scales from the first
//   dwords of chunks 0 and 2. So a slice of the reduction starts on an even k-block and the rows
//   hold an even number of blocks (the host sends other Q8_0 shapes to matmul.hip).
#include "common.h"

namespace {

constexpr uint32_t MM2_TOK = 128;   // tokens per work-group
constexpr uint32_t MM2_ROWS = 128;  // weight rows per work-group (the wide form: 256)
constexpr uint32_t MM2_HALF = MM2_TOK * 64u;    // bytes of one half (hi or lo) of an activation tile
constexpr uint32_t MM2_ACT = 2u * MM2_HALF;     // one k-block's activation tile
constexpr uint32_t MM2_NBUF = 3u;
// Q8_0 pair buffer (mm2_body's QPAIR): the rows' 64-byte pieces, their tails (rows 0 .. 63 from
// wave 0, 64 .. 127 from wave 1, ...), and 256 bytes per remaining wave that it fills with the same
// tails as the wave it repeats (so every wave issues the same copies; nothing reads them)

// Q4_K, Q5_K (per work-group, after the activation buffers): the k-blocks' per-token block sums
// (128 floats, three buffers), each pair of sub-blocks' 32 payload bytes per row (the low nibbles
// are the pair's first sub-block, the high ones its second; three buffers) and each super-block's
// header per row (d, dmin, the 12 scale bytes; Q5_K: and the 32 bytes of fifth bits; two buffers)
constexpr uint32_t MM2_KXS = MM2_TOK * 4u;
// (The per-row buffers' sizes follow the tile's row count: mm2_body's KPAIR_B, KHDR_B, QUAD6_B,
// HDR6_B and XPAIR_B.)
// Q6_K (per work-group, after the activation buffers): each half super-block's (four k-blocks')
// 64 bytes of ql and 32 of qh per row (two buffers), and each super-block's 16 scale bytes per row
// followed by a dword per row ending on d (bytes 206 .. 209; two buffers)
// MXFP4 (per work-group, after the activation buffers): each pair of 17-byte blocks' 34 bytes per
// row, as two 16-byte chunks (bytes 0 .. 31) and a 4-byte tail (bytes 30 .. 33, which ends on the
// pair's last byte, so no copy reads past a row); three buffers

typedef float mm2_f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t mm2_u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t mm2_swz(uint32_t t) { return (t >> 2) & 3u; }

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

// 8 nibbles (one per byte, values 0 .. 15) in two dwords -> 8 exact f16: under exponent 0x64 the
// byte is 1024 + q
__device__ __forceinline__ half8_t mm2_u4_to_f16(mm2_u32x2 q) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, q[i], 0x04010400u);
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, q[i], 0x04030402u);
        const half2_t h0 = __builtin_bit_cast(half2_t, p0) - half2_t{(_Float16) 1024.f, (_Float16) 1024.f};
        const half2_t h1 = __builtin_bit_cast(half2_t, p1) - half2_t{(_Float16) 1024.f, (_Float16) 1024.f};
        r[4 * i] = h0[0];
        r[4 * i + 1] = h0[1];
        r[4 * i + 2] = h1[0];
        r[4 * i + 3] = h1[1];
    }
    return r;
}

// The same for 6-bit values q + 32 (0 .. 63) -> exact f16 q in [-32, 31]
__device__ __forceinline__ half8_t mm2_u6_to_f16(mm2_u32x2 q) {
    half8_t r;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, q[i], 0x04010400u);
        const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, q[i], 0x04030402u);
        const half2_t h0 = __builtin_bit_cast(half2_t, p0) - half2_t{(_Float16) 1056.f, (_Float16) 1056.f};
        const half2_t h1 = __builtin_bit_cast(half2_t, p1) - half2_t{(_Float16) 1056.f, (_Float16) 1056.f};
        r[4 * i] = h0[0];
        r[4 * i + 1] = h0[1];
        r[4 * i + 2] = h1[0];
        r[4 * i + 3] = h1[1];
    }
    return r;
}

// LDS-DMA copies of 16 (or 4) bytes per lane from src to LDS byte lds + 16 lane (4 lane). Issued as
// asm (m0 saved and restored, memory clobbered), out of the compiler's wait bookkeeping: with such
// copies in flight it would drain every memory operation (vmcnt(0)) before each step's LDS reads,
// the copies just requested for two blocks ahead included. The step's leading wait covers them.
__device__ __forceinline__ void mm2_copy16(uint32_t lds, const void *src) {
    uint32_t m0_saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(m0_saved)
                 : "s"(lds), "v"(src)
                 : "memory");
}
__device__ __forceinline__ void mm2_copy4(uint32_t lds, const void *src) {
    uint32_t m0_saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dword %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(m0_saved)
                 : "s"(lds), "v"(src)
                 : "memory");
}

__device__ __forceinline__ u32x4_t mm2_lds16(uint32_t off) {
    return *(const __attribute__((address_space(3))) u32x4_t *) (uintptr_t) off;
}
__device__ __forceinline__ uint32_t mm2_lds4(uint32_t off) {
    return *(const __attribute__((address_space(3))) uint32_t *) (uintptr_t) off;
}

template <uint32_t TY, bool WIDE = false>
__device__ __forceinline__ void mm2_body(const MatmulArgs &a) {
    constexpr bool Q8 = TY == 8, Q4K = TY == 12 || TY == 13, Q5K = TY == 13, Q6K = TY == 14, MX = TY == 39;
    constexpr uint32_t KSB = Q5K ? 176u : 144u, KQS = Q5K ? 48u : 16u;  // super-block bytes, qs offset
    // WIDE: eight waves over 128 tokens x 256 rows, one work-group per CU; the per-wave tiles and
    // steps are the same, each k-block's copies are shared by twice the rows. The K-quants, built
    // this way (their per-row buffers and header copies below follow ROWS and RQ), measured no gain
    // (Q4_K, Q5_K within noise, Q6_K 6% slower): the two waves of a SIMD then belong to one
    // work-group and meet at every barrier, and in their VALU-heavy steps they contend where two
    // work-groups' waves would interleave.
    static_assert(!WIDE || TY == 1 || TY == 8 || TY == 39, "wide tiles: F16, Q8_0 and MXFP4");
    constexpr uint32_t NW = WIDE ? 8u : 4u;                 // waves
    constexpr uint32_t ROWS = WIDE ? 2u * MM2_ROWS : MM2_ROWS;  // weight rows per work-group
    constexpr uint32_t RQ = ROWS / 64u;                     // 64-row quarters: per-row copies by waves w % RQ
    constexpr uint32_t NAI = 16u / NW;                      // activation copies per wave and step
    constexpr uint32_t QTAIL = ROWS * 64u, QPAIR = QTAIL + NW * 256u;
    // the per-row weight buffers at this tile's row count
    constexpr uint32_t KPAIR_B = ROWS * 32u, KHDR_B = ROWS * (Q5K ? 48u : 16u);
    constexpr uint32_t QUAD6_B = ROWS * 96u, HDR6_B = ROWS * 20u, XPAIR_B = ROWS * 36u;
    // LDS: per buffer a k-block's activation tile and (F16) its weight tile; then (Q8_0) the pair
    // buffers, (Q4_K) the block sums, pair and header buffers
    constexpr uint32_t BUF = MM2_ACT + (TY == 1 ? ROWS * 64u : 0u);
    constexpr uint32_t QBASE = MM2_NBUF * BUF;
    constexpr uint32_t KXS = QBASE, KPAIR = KXS + MM2_NBUF * MM2_KXS, KHDR = KPAIR + MM2_NBUF * KPAIR_B;
    constexpr uint32_t K6Q = QBASE, K6H = K6Q + 2u * QUAD6_B;
    constexpr uint32_t EXTRA = Q8 ? MM2_NBUF * QPAIR : Q4K ? KHDR - QBASE + 2u * KHDR_B
                             : Q6K ? 2u * QUAD6_B + 2u * HDR6_B : MX ? MM2_NBUF * XPAIR_B : 0u;
    __shared__ __attribute__((aligned(1024))) uint8_t tiles[QBASE + EXTRA];
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n = lane & 31u, h = lane >> 5;
    const MmSegView sg = mm_seg(a, blockIdx.x);
    const uint32_t t0 = blockIdx.y * MM2_TOK, r0 = sg.tile * ROWS;
    // this work-group's k-slice: blocks kb0 .. kb0 + nb (Q8_0: both even)
    const uint32_t kb0 = blockIdx.z * a.kb_per, nb = min(a.kb_per, a.cols / 32u - kb0);
    const uint32_t lds0 =
        __builtin_amdgcn_readfirstlane((uint32_t) (uintptr_t) (__attribute__((address_space(3))) uint8_t *) tiles);

    // Activation copies: instruction i of wave w fills region R = NAI w + i (1 KiB): half R >> 3,
    // tokens 16 (R & 7) .. + 15; lane L writes slot L of the region = chunk position L & 3 of token
    // L >> 2, which holds chunk (L & 3) ^ swz(token).
    const uint16_t *xsrc[NAI];
#pragma unroll
    for (int i = 0; i < (int) NAI; ++i) {
        const uint32_t R = NAI * wave + (uint32_t) i;
        const uint32_t tok = 16u * (R & 7u) + (lane >> 2);
        const uint32_t c = (lane & 3u) ^ mm2_swz(tok);
        const uint64_t tg = min(t0 + tok, a.n_tok - 1u);
        xsrc[i] = ((R >> 3) ? a.xl : a.xh) + tg * a.cols + 32u * kb0 + 8u * c;
    }
    // Weight copies: instruction i of wave w fills rows 16 (2 w + i) .. + 15 of the 64-byte pieces
    // (F16: one k-block; Q8_0: bytes 0 .. 63 of a pair), lane L row 16 (2 w + i) + (L >> 2), whose
    // position L & 3 holds chunk (L & 3) ^ swz(row); Q8_0: wave w also copies the tails of rows
    // 64 (w & 1) .. + 63 (lane L: row 64 (w & 1) + L; wide: 64 (w & 3) + L, waves 4-7 repeating
    // 0-3 into slots nothing reads). Rows past the last copy the last row (not stored).
    constexpr uint32_t wbb = Q8 ? 34u : 64u;  // bytes of a row per k-block
    const uint8_t *wsrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t rl = 16u * (2u * wave + (uint32_t) i) + (lane >> 2);
        wsrc[i] = sg.w + (uint64_t) min(r0 + rl, sg.rows - 1u) * sg.row_bytes + wbb * (uint64_t) kb0 +
                  16u * ((lane & 3u) ^ mm2_swz(rl));
    }
    const uint8_t *wtail =
        sg.w + (uint64_t) min(r0 + 64u * (wave % (ROWS / 64u)) + lane, sg.rows - 1u) * sg.row_bytes + 34u * (uint64_t) kb0 + 64u;

    // block b's activations (F16: and weights) into buffer buf
    auto copy = [&](uint32_t b, uint32_t buf) {
#pragma unroll
        for (int i = 0; i < (int) NAI; ++i)
            mm2_copy16(__builtin_amdgcn_readfirstlane(lds0 + buf * BUF + (NAI * wave + (uint32_t) i) * 1024u),
                       xsrc[i] + 32u * b);
        if constexpr (TY == 1) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
                mm2_copy16(__builtin_amdgcn_readfirstlane(lds0 + buf * BUF + MM2_ACT + (2u * wave + (uint32_t) i) * 1024u),
                           wsrc[i] + 64u * b);
        }
    };
    // Q4_K: per k-block b (into buffers buf, qb and the header buffer of b's super-block) the block
    // sums of the tile's tokens, b's pair of sub-blocks, b's super-block header -- three copies for
    // every block, whichever of them repeat the previous block's bytes, so each step issues the
    // same count. Waves from 2 on copy the same sums as waves 0 and 1, waves from RQ on the same
    // headers as waves 0 .. RQ - 1 (the same bytes to the same places). Pair slot q = 64 wave + lane
    // holds row q / 2's 16-byte chunk (q & 1) ^ ((row >> 3) & 1) of the pair's 32 payload bytes
    // (qs[32 g .. 32 g + 31]).
    const uint32_t k_row = (64u * wave + lane) >> 1;
    const uint8_t *k_psrc = sg.w + (uint64_t) min(r0 + k_row, sg.rows - 1u) * sg.row_bytes + KQS +
                            16u * ((lane & 1u) ^ ((k_row >> 3) & 1u));
    const uint8_t *k_hsrc = sg.w + (uint64_t) min(r0 + 64u * (wave % RQ) + lane, sg.rows - 1u) * sg.row_bytes;
    const float *k_xsrc = a.xs + (uint64_t) min(t0 + 64u * (wave & 1u) + lane, a.n_tok - 1u) * (a.cols / 32u) + kb0;
    // Q5_K header slots: instruction i of wave w fills slots 64 s .. + 63, s = min(2 w + i, 3 RQ - 1)
    // (the last waves repeat the last 64 slots); slot q is row q / 3's 16-byte chunk q % 3
    auto k5slot = [&](uint32_t i) { return 64u * min(2u * wave + i, 3u * RQ - 1u); };
    const uint8_t *k5hsrc[2];
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i) {
        const uint32_t q = k5slot(i) + lane;
        k5hsrc[i] = sg.w + (uint64_t) min(r0 + q / 3u, sg.rows - 1u) * sg.row_bytes + 16u * (q % 3u);
    }
    auto kcopy = [&](uint32_t b, uint32_t buf, uint32_t qb) {
        const uint32_t kb = kb0 + b;  // super-block kb / 8, pair (kb % 8) / 2
        mm2_copy4(__builtin_amdgcn_readfirstlane(lds0 + KXS + buf * MM2_KXS + (wave & 1u) * 256u), k_xsrc + b);
        mm2_copy16(__builtin_amdgcn_readfirstlane(lds0 + KPAIR + qb * KPAIR_B + wave * 1024u),
                   k_psrc + KSB * (uint64_t) (kb >> 3) + 32u * ((kb & 7u) >> 1));
        const uint32_t hbase = lds0 + KHDR + ((b >> 3) & 1u) * KHDR_B;
        if constexpr (Q5K) {
#pragma unroll
            for (uint32_t i = 0; i < 2; ++i)
                mm2_copy16(__builtin_amdgcn_readfirstlane(hbase + 16u * k5slot(i)), k5hsrc[i] + KSB * (uint64_t) (kb >> 3));
        } else {
            mm2_copy16(__builtin_amdgcn_readfirstlane(hbase + (wave % RQ) * 1024u), k_hsrc + KSB * (uint64_t) (kb >> 3));
        }
    };
    // Q8_0: the weights of blocks b, b + 1 (b even) into pair buffer qb
    auto qcopy = [&](uint32_t b, uint32_t qb) {
        const uint32_t base = lds0 + QBASE + qb * QPAIR;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            mm2_copy16(__builtin_amdgcn_readfirstlane(base + (2u * wave + (uint32_t) i) * 1024u), wsrc[i] + 34u * b);
        mm2_copy4(__builtin_amdgcn_readfirstlane(base + QTAIL + wave * 256u), wtail + 34u * b);
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
            // Q6_K: slice s holds one 16-wide scale group, k 16 s + 8 h .. + 7, chunk 2 s + h
            const uint32_t ch = Q6K ? 2u * s + h : 2u * h + s;
            aoff[tt][s] = lds0 + tok * 64u + 16u * (ch ^ mm2_swz(tok));
        }
    // B operand (weights) of row tile rt: row 64 (w >> 1) + 32 rt + n. F16 slice s: chunk 2 h + s.
    // Q8_0 (pair buffer 0): [0] chunk h, [1] chunk h + 1, [2] chunk h + 2, [3] chunk 3 (h = 0) or the
    // tail (h = 1), [4] chunk 0, [5] chunk 2.
    uint32_t woff[2][Q8 ? 6 : 2];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
        const uint32_t rl = 64u * (wave >> 1) + 32u * rt + n;
        const uint32_t sw = mm2_swz(rl);
        if constexpr (Q8) {
            const uint32_t base = lds0 + QBASE + rl * 64u;
            woff[rt][0] = base + 16u * (h ^ sw);
            woff[rt][1] = base + 16u * ((h + 1u) ^ sw);
            woff[rt][2] = base + 16u * ((h + 2u) ^ sw);
            woff[rt][3] = h ? lds0 + QBASE + QTAIL + rl * 4u : base + 16u * (3u ^ sw);
            woff[rt][4] = base + 16u * sw;
            woff[rt][5] = base + 16u * (2u ^ sw);
        } else {
#pragma unroll
            for (int s = 0; s < 2; ++s) woff[rt][s] = lds0 + MM2_ACT + rl * 64u + 16u * ((2u * h + s) ^ sw);
        }
    }

    // Q6_K: per k-block b (into the buffers of b's half super-block and super-block) its half
    // super-block's ql and qh (128 rows x six 16-byte chunks: slot q = 192 i + 64 wave... holds row
    // q / 6's chunk q % 6, three copies a lane) and its super-block's scales and d (a 16-byte copy
    // and a dword copy per row: waves 2 and 3 repeat waves 0 and 1) -- every block, whichever of them
    // repeat the previous block's bytes, so each step issues the same five copies
    // (each lane's three chunk sources within super-block 0 and their step per half super-block)
    const uint8_t *k6src[3];
    uint32_t k6hstep[3];
#pragma unroll
    for (uint32_t i = 0; i < 3; ++i) {
        const uint32_t q = 64u * (NW * i + wave) + lane, r = q / 6u, c = q % 6u;  // ql chunks 0 .. 3, qh 4, 5
        k6src[i] = sg.w + (uint64_t) min(r0 + r, sg.rows - 1u) * sg.row_bytes + 210u * (uint64_t) (kb0 >> 3) +
                   (c < 4u ? 16u * c : 128u + 16u * (c - 4u));
        k6hstep[i] = c < 4u ? 64u : 32u;
    }
    auto k6copy = [&](uint32_t b) {
        const uint32_t kb = kb0 + b;  // super-block kb / 8, half (kb % 8) / 4
        const uint64_t sbo = 210u * (uint64_t) (b >> 3);
        const uint32_t qbase = lds0 + K6Q + ((b >> 2) & 1u) * QUAD6_B;
#pragma unroll
        for (uint32_t i = 0; i < 3; ++i)
            mm2_copy16(__builtin_amdgcn_readfirstlane(qbase + 16u * (64u * (NW * i + wave))),
                       k6src[i] + sbo + ((kb >> 2) & 1u) * k6hstep[i]);
        const uint32_t hbase = lds0 + K6H + ((b >> 3) & 1u) * HDR6_B;
        const uint8_t *hrow = k_hsrc + 210u * (uint64_t) (kb >> 3);
        mm2_copy16(__builtin_amdgcn_readfirstlane(hbase + (wave % RQ) * 1024u), hrow + 192u);
        mm2_copy4(__builtin_amdgcn_readfirstlane(hbase + ROWS * 16u + (wave % RQ) * 256u), hrow + 206u);
    };
    // MXFP4: per k-block b the pair (b's and its partner's 34 bytes per row) into pair buffer qb --
    // every block, the odd one repeating the even one's bytes, so each step issues the same two
    // copies. Chunk slot q = 64 wave + lane holds row q / 2's chunk (q & 1) ^ ((row >> 3) & 1); the
    // tails (rows 64 (wave & 1) + lane) sit after the 128 rows' chunks, waves 2 and 3 repeating
    // waves 0 and 1.
    const uint8_t *x_csrc = sg.w + (uint64_t) min(r0 + k_row, sg.rows - 1u) * sg.row_bytes + 17u * (uint64_t) kb0 +
                            16u * ((lane & 1u) ^ ((k_row >> 3) & 1u));
    const uint8_t *x_tsrc = sg.w + (uint64_t) min(r0 + 64u * (wave % RQ) + lane, sg.rows - 1u) * sg.row_bytes +
                            17u * (uint64_t) kb0 + 30u;
    auto xcopy = [&](uint32_t b, uint32_t qb) {
        const uint64_t po = 34u * (uint64_t) (b >> 1);
        mm2_copy16(__builtin_amdgcn_readfirstlane(lds0 + QBASE + qb * XPAIR_B + wave * 1024u), x_csrc + po);
        mm2_copy4(__builtin_amdgcn_readfirstlane(lds0 + QBASE + qb * XPAIR_B + ROWS * 32u + (wave % RQ) * 256u),
                  x_tsrc + po);
    };
    // block b from activation buffer buf and (Q8_0, Q4_K) pair buffer qb, b odd: the pair's second block
    auto compute = [&](uint32_t buf, uint32_t qb, bool odd, uint32_t b) {
        half8_t ah[2][2], al[2][2], bw[2][2];
        float d[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const uint32_t off = aoff[tt][s] + buf * BUF;
                ah[tt][s] = __builtin_bit_cast(half8_t, mm2_lds16(off));
                al[tt][s] = __builtin_bit_cast(half8_t, mm2_lds16(off + MM2_HALF));
            }
        if constexpr (MX) {
            // block (odd: the pair's second) of 17 bytes: E8M0 exponent e, then element j in the low
            // nibble of data byte j and element j + 16 in its high nibble. This lane's k are
            // 16 h .. 16 h + 15: the low (h = 0) or high (h = 1) nibbles of all 16 data bytes.
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const uint32_t rl = 64u * (wave >> 1) + 32u * rt + n;
                const uint32_t prow = lds0 + QBASE + qb * XPAIR_B;
                const uint32_t sw = (rl >> 3) & 1u;
                const u32x4_t c0 = mm2_lds16(prow + 32u * rl + 16u * sw);          // bytes 0 .. 15
                const u32x4_t c1 = mm2_lds16(prow + 32u * rl + 16u * (1u ^ sw));   // bytes 16 .. 31
                const uint32_t tl = mm2_lds4(prow + ROWS * 32u + 4u * rl);     // bytes 30 .. 33
                uint32_t dw[4], e;
                if (!odd) {  // data bytes 1 .. 16
                    dw[0] = __builtin_amdgcn_alignbyte(c0[1], c0[0], 1u);
                    dw[1] = __builtin_amdgcn_alignbyte(c0[2], c0[1], 1u);
                    dw[2] = __builtin_amdgcn_alignbyte(c0[3], c0[2], 1u);
                    dw[3] = __builtin_amdgcn_alignbyte(c1[0], c0[3], 1u);
                    e = c0[0] & 0xFFu;
                } else {  // data bytes 18 .. 33
                    dw[0] = __builtin_amdgcn_alignbyte(c1[1], c1[0], 2u);
                    dw[1] = __builtin_amdgcn_alignbyte(c1[2], c1[1], 2u);
                    dw[2] = __builtin_amdgcn_alignbyte(c1[3], c1[2], 2u);
                    dw[3] = __builtin_amdgcn_alignbyte(tl >> 16, c1[3], 2u);
                    e = (c1[0] >> 8) & 0xFFu;
                }
                d[rt] = __uint_as_float(e ? e << 23 : 0x00400000u);  // 2^(e - 127)
                // codes of elements (16 h + 4 i ..): nibble h of the dword's bytes, paired into bytes
                // 0 and 2 as (element, next element) for the two-value conversions
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    half8_t v;
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        const uint32_t x = (dw[2 * s + i] >> (4u * h)) & 0x0F0F0F0Fu;
                        const uint32_t y = x | (x >> 4);
                        const half2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(y, 1.0f, 0);
                        const half2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(y, 1.0f, 2);
                        v[4 * i] = p0[0];
                        v[4 * i + 1] = p0[1];
                        v[4 * i + 2] = p1[0];
                        v[4 * i + 3] = p1[1];
                    }
                    bw[rt][s] = v;
                }
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    mm2_f32x16 sblk = {};
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        sblk = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tt][s], bw[rt][s], sblk, 0, 0, 0);
                        sblk = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tt][s], bw[rt][s], sblk, 0, 0, 0);
                    }
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[tt][rt][j] = fmaf(d[rt], sblk[j], acc[tt][rt][j]);
                }
            return;
        }
        if constexpr (Q6K) {
            // k-block c of half super-block hf: low four bits from ql[64 hf + 32 (c & 1) + l]
            // (nibble c >> 1), high two from qh[32 hf + l] (bits 2c, 2c + 1), l the element; this
            // lane's slice s holds l = 16 s + 8 h .. + 7 (scale group s)
            const uint32_t kb = kb0 + b, c = kb & 3u, hf = (kb >> 2) & 1u;
            const uint32_t shl = 4u * (c >> 1), shh = 2u * c;
            float ds[2][2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const uint32_t rl = 64u * (wave >> 1) + 32u * rt + n;
                const uint32_t qrow = lds0 + K6Q + ((b >> 2) & 1u) * QUAD6_B + 96u * rl;
                const uint32_t hbase = lds0 + K6H + ((b >> 3) & 1u) * HDR6_B;
                const uint32_t scw = *(const __attribute__((address_space(3))) uint32_t *) (uintptr_t) (
                    hbase + 16u * rl + 4u * (2u * hf + (c >> 1)));  // scales[8 hf + 2c], + 1
                const uint32_t dw = *(const __attribute__((address_space(3))) uint32_t *) (uintptr_t) (
                    hbase + ROWS * 16u + 4u * rl);
                const float d = (float) __builtin_bit_cast(_Float16, (uint16_t) (dw >> 16));
                const uint32_t sco = 16u * (c & 1u);
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2) ds[rt][s2] = d * (float) (int8_t) (uint8_t) (scw >> (sco + 8u * (uint32_t) s2));
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const mm2_u32x2 ql = *(const __attribute__((address_space(3))) mm2_u32x2 *) (uintptr_t) (
                        qrow + 16u * (2u * (c & 1u) + (uint32_t) s) + 8u * h);
                    const mm2_u32x2 qh = *(const __attribute__((address_space(3))) mm2_u32x2 *) (uintptr_t) (
                        qrow + 64u + 16u * (uint32_t) s + 8u * h);
                    const uint32_t w0 = ((ql[0] >> shl) & 0x0F0F0F0Fu) | (((qh[0] >> shh) & 0x03030303u) << 4);
                    const uint32_t w1 = ((ql[1] >> shl) & 0x0F0F0F0Fu) | (((qh[1] >> shh) & 0x03030303u) << 4);
                    bw[rt][s] = mm2_u6_to_f16(mm2_u32x2{w0, w1});
                }
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    mm2_f32x16 sg0 = {}, sg1 = {};
                    sg0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tt][0], bw[rt][0], sg0, 0, 0, 0);
                    sg0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tt][0], bw[rt][0], sg0, 0, 0, 0);
                    sg1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tt][1], bw[rt][1], sg1, 0, 0, 0);
                    sg1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tt][1], bw[rt][1], sg1, 0, 0, 0);
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        acc[tt][rt][j] = fmaf(ds[rt][1], sg1[j], fmaf(ds[rt][0], sg0[j], acc[tt][rt][j]));
                }
            return;
        }
        if constexpr (Q4K) {
            // this lane's 16 payload bytes of the pair (its k of both sub-blocks) and the
            // super-block header (d, dmin, 12 scale bytes) of each row tile: both stay in their
            // buffers for every step that reads them
            const uint32_t sb = b & 7u;  // sub-block within the super-block (slices start on one)
            float d1[2], m1[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const uint32_t rl = 64u * (wave >> 1) + 32u * rt + n;
                const u32x4_t kq = mm2_lds16(lds0 + KPAIR + qb * KPAIR_B + 32u * rl + 16u * (h ^ ((rl >> 3) & 1u)));
                const uint32_t hrow = lds0 + KHDR + ((b >> 3) & 1u) * KHDR_B + (Q5K ? 48u : 16u) * rl;
                const u32x4_t hd = mm2_lds16(hrow);
                // get_scale_min_k4 (reference.rs:150-160) over the 12 scale bytes hd.y .. hd.w
                // (a mask, not a branch or a select: those split the step and its registers spill)
                const uint32_t i = 8u * (sb & 3u);
                const uint32_t a1 = hd[1] >> i, a2 = hd[2] >> i, a3 = hd[3] >> i;
                const uint32_t lo = sb < 4u ? ~0u : 0u;  // uniform
                const uint32_t sc = ((a1 & 63u) & lo) | (((a3 & 15u) | (((a1 >> 6) & 3u) << 4)) & ~lo);
                const uint32_t mn = ((a2 & 63u) & lo) | ((((a3 >> 4) & 15u) | (((a2 >> 6) & 3u) << 4)) & ~lo);
                d1[rt] = (float) __builtin_bit_cast(_Float16, (uint16_t) (hd[0] & 0xFFFFu)) * (float) sc;
                m1[rt] = (float) __builtin_bit_cast(_Float16, (uint16_t) (hd[0] >> 16)) * (float) mn;
                const uint32_t sh = odd ? 4u : 0u;  // the pair's first sub-block: low nibbles
                // Q5_K: element e's fifth bit is bit sb of qh[e]; this lane's elements 16 h ..
                // + 15 have qh[16 h .. 16 h + 15], the header's chunk 1 + h
                u32x4_t qh = {};
                if constexpr (Q5K) qh = mm2_lds16(hrow + 16u + 16u * h);
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    uint32_t w0 = (kq[2 * s] >> sh) & 0x0F0F0F0Fu, w1 = (kq[2 * s + 1] >> sh) & 0x0F0F0F0Fu;
                    if constexpr (Q5K) {
                        w0 |= ((qh[2 * s] >> sb) & 0x01010101u) << 4;
                        w1 |= ((qh[2 * s + 1] >> sb) & 0x01010101u) << 4;
                    }
                    bw[rt][s] = mm2_u4_to_f16(mm2_u32x2{w0, w1});
                }
            }
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                // the block sums of this lane's accumulators: element j is token 8 (j / 4) + 4 h + j % 4
                float4_t xs[4];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    xs[q] = *(const __attribute__((address_space(3))) float4_t *) (uintptr_t) (
                        lds0 + KXS + buf * MM2_KXS + 4u * (64u * (wave & 1u) + 32u * tt + 8u * q + 4u * h));
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    mm2_f32x16 sblk = {};
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        sblk = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tt][s], bw[rt][s], sblk, 0, 0, 0);
                        sblk = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tt][s], bw[rt][s], sblk, 0, 0, 0);
                    }
                    // d1 * (sum q x) - m1 * (sum x): the reference's sub-block regrouped
#pragma unroll
                    for (int j = 0; j < 16; ++j)
                        acc[tt][rt][j] = fmaf(-m1[rt], xs[j >> 2][j & 3], fmaf(d1[rt], sblk[j], acc[tt][rt][j]));
                }
            }
            return;
        }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            if constexpr (Q8) {
                const uint32_t qo = qb * QPAIR;
                u32x4_t q;
                uint32_t dd;
                if (!odd) {  // window bytes 2 + 16h .. 17 + 16h
                    const u32x4_t c = mm2_lds16(woff[rt][0] + qo);
                    const uint32_t nx = mm2_lds4(woff[rt][1] + qo);
                    q = (u32x4_t){__builtin_amdgcn_alignbyte(c[1], c[0], 2u), __builtin_amdgcn_alignbyte(c[2], c[1], 2u),
                                  __builtin_amdgcn_alignbyte(c[3], c[2], 2u), __builtin_amdgcn_alignbyte(nx, c[3], 2u)};
                    dd = mm2_lds4(woff[rt][4] + qo) & 0xFFFFu;
                } else {  // window bytes 36 + 16h .. 51 + 16h
                    const u32x4_t c = mm2_lds16(woff[rt][2] + qo);
                    q = (u32x4_t){c[1], c[2], c[3], mm2_lds4(woff[rt][3] + qo)};
                    dd = mm2_lds4(woff[rt][5] + qo) >> 16;
                }
                d[rt] = (float) __builtin_bit_cast(_Float16, (uint16_t) dd);
#pragma unroll
                for (int s = 0; s < 2; ++s) bw[rt][s] = mm2_i8_to_f16(mm2_u32x2{q[2 * s], q[2 * s + 1]});
            } else {
#pragma unroll
                for (int s = 0; s < 2; ++s) bw[rt][s] = __builtin_bit_cast(half8_t, mm2_lds16(woff[rt][s] + buf * BUF));
            }
        }
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                if constexpr (Q8) {
                    mm2_f32x16 sblk = {};
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        sblk = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tt][s], bw[rt][s], sblk, 0, 0, 0);
                        sblk = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tt][s], bw[rt][s], sblk, 0, 0, 0);
                    }
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[tt][rt][j] = fmaf(d[rt], sblk[j], acc[tt][rt][j]);
                } else {
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        acc[tt][rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[tt][s], bw[rt][s], acc[tt][rt], 0, 0, 0);
                        acc[tt][rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[tt][s], bw[rt][s], acc[tt][rt], 0, 0, 0);
                    }
                }
            }
    };

    // k-block b's activations in buffer b % 3 (F16: its weights beside them); Q8_0: pair b / 2 in
    // pair buffer (b / 2) % 3. Step b: wait for block b's copies (b even, Q8_0: and its pair's), meet
    // the other waves (every wave has finished block b - 1, whose buffers are refilled next),
    // request block b + 2 (Q8_0, b even: and pair b + 2, b + 3), compute block b. A wave issues NAI
    // activation copies per block (4; 2 in the wide form), F16 two weight copies beside them, Q8_0
    // three pair copies after every even block's. Copies that may stay in flight at step b: F16,
    // block b + 1's (NAI + 2); Q8_0, b even: block b + 1's activations (NAI); b odd: block b + 1's
    // activations and pair b + 1's weights (NAI + 3). Past the end, the requests repeat the last
    // block and pair into the buffers next in line, which nothing reads, so every step issues the
    // same copies.
    if constexpr (WIDE && TY == 1) {
        // Register pipeline (F16, wide): step b reads block b + 1's operands from LDS into registers
        // while block b's MFMAs run on the operands read one step earlier, and requests block b + 3
        // into the buffer block b has left. (In the wide form the two waves of a SIMD belong to one
        // work-group and meet at every barrier, so neither covers the other's wait for its reads.)
        constexpr uint32_t PER = NAI + 2u;  // copies per step
        struct Ops {
            half8_t ah[2][2], al[2][2], bw[2][2];
        };
        auto rd = [&](uint32_t buf) {
            Ops o;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const uint32_t off = aoff[tt][s] + buf * BUF;
                    o.ah[tt][s] = __builtin_bit_cast(half8_t, mm2_lds16(off));
                    o.al[tt][s] = __builtin_bit_cast(half8_t, mm2_lds16(off + MM2_HALF));
                }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int s = 0; s < 2; ++s) o.bw[rt][s] = __builtin_bit_cast(half8_t, mm2_lds16(woff[rt][s] + buf * BUF));
            return o;
        };
        auto mm = [&](const Ops &o) {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        acc[tt][rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(o.ah[tt][s], o.bw[rt][s], acc[tt][rt], 0, 0, 0);
                        acc[tt][rt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(o.al[tt][s], o.bw[rt][s], acc[tt][rt], 0, 0, 0);
                    }
        };
        // blocks 0, 1, 2 requested; block 0's have landed everywhere
        copy(0u, 0u);
        copy(min(1u, nb - 1u), 1u);
        copy(min(2u, nb - 1u), 2u);
        __builtin_amdgcn_s_waitcnt(mm2_vmcnt(2u * PER));
        __builtin_amdgcn_s_barrier();
        Ops cur = rd(0u);
        // step b (buffer of block b: i = b % 3): block b + 1's copies have landed and every LDS read
        // of block b has returned, in this wave, then in every wave
        auto pstep = [&](uint32_t b, uint32_t i) {
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(mm2_vmcnt_lgkm0(PER));
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            const Ops nxt = rd((i + 1u) % 3u);
            copy(min(b + 3u, nb - 1u), i);
            __builtin_amdgcn_sched_barrier(0);
            mm(cur);
            cur = nxt;
        };
        uint32_t b = 0;
        for (; b + 3u <= nb; b += 3u) {
            pstep(b, 0u);
            pstep(b + 1u, 1u);
            pstep(b + 2u, 2u);
        }
        if (b < nb) pstep(b, 0u);
        if (b + 1u < nb) pstep(b + 1u, 1u);
        __builtin_amdgcn_s_waitcnt(mm2_vmcnt(0));  // no copy outlives the work-group
    } else {
    copy(0, 0);
    if constexpr (Q8) qcopy(0, 0);
    if constexpr (Q4K) kcopy(0, 0, 0);
    if constexpr (Q6K) k6copy(0);
    if constexpr (MX) xcopy(0, 0);
    copy(min(1u, nb - 1u), 1);
    if constexpr (Q4K) kcopy(min(1u, nb - 1u), 1, 0);
    if constexpr (Q6K) k6copy(min(1u, nb - 1u));
    if constexpr (MX) xcopy(min(1u, nb - 1u), 0);
    auto step = [&](uint32_t b, uint32_t buf, uint32_t qb, bool odd) {
        // block b's copies have landed and every LDS read of block b - 1 has returned, in this wave;
        // then in every wave
        __builtin_amdgcn_sched_barrier(0);
        if (Q6K)
            __builtin_amdgcn_s_waitcnt(mm2_vmcnt_lgkm0(NAI + 5u));  // NAI + 3 quads + header 2
        else if (Q5K)
            __builtin_amdgcn_s_waitcnt(mm2_vmcnt_lgkm0(NAI + 4u));  // NAI + sums + pair + header 2
        else if (Q4K)
            __builtin_amdgcn_s_waitcnt(mm2_vmcnt_lgkm0(NAI + 3u));  // NAI + sums + pair + header
        else if (!Q8)
            __builtin_amdgcn_s_waitcnt(mm2_vmcnt_lgkm0(NAI + 2u));  // F16: NAI + 2 copies; MXFP4: 4 + 2
        else if (odd)
            __builtin_amdgcn_s_waitcnt(mm2_vmcnt_lgkm0(NAI + 3u));
        else
            __builtin_amdgcn_s_waitcnt(mm2_vmcnt_lgkm0(NAI));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        copy(min(b + 2u, nb - 1u), (buf + 2u) % 3u);
        if constexpr (Q8)
            if (!odd) qcopy(min(b + 2u, nb - 2u), (qb + 1u) % 3u);
        if constexpr (Q4K) kcopy(min(b + 2u, nb - 1u), (buf + 2u) % 3u, (qb + 1u) % 3u);
        if constexpr (Q6K) k6copy(min(b + 2u, nb - 1u));
        if constexpr (MX) xcopy(min(b + 2u, nb - 1u), (qb + 1u) % 3u);
        __builtin_amdgcn_sched_barrier(0);
        compute(buf, qb, odd, b);
    };
    uint32_t b = 0;
    for (; b + 6u <= nb; b += 6u) {
        step(b, 0, 0, false);
        step(b + 1u, 1, 0, true);
        step(b + 2u, 2, 1, false);
        step(b + 3u, 0, 1, true);
        step(b + 4u, 1, 2, false);
        step(b + 5u, 2, 2, true);
    }
    if (b < nb) step(b, 0, 0, false);
    if (b + 1u < nb) step(b + 1u, 1, 0, true);
    if (b + 2u < nb) step(b + 2u, 2, 1, false);
    if (b + 3u < nb) step(b + 3u, 0, 1, true);
    if (b + 4u < nb) step(b + 4u, 1, 2, false);
    __builtin_amdgcn_s_waitcnt(mm2_vmcnt(0));  // no copy outlives the work-group
    }

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
extern "C" __global__ void __launch_bounds__(512) moearc_matmul2w_q8_0_k(MatmulArgs a) { mm2_body<8, true>(a); }
extern "C" __global__ void __launch_bounds__(512) moearc_matmul2w_f16_k(MatmulArgs a) { mm2_body<1, true>(a); }
extern "C" __global__ void __launch_bounds__(512) moearc_matmul2w_mxfp4_k(MatmulArgs a) { mm2_body<39, true>(a); }
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
moearc_matmul2_q4_k_k(MatmulArgs a) { mm2_body<12>(a); }
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
moearc_matmul2_q5_k_k(MatmulArgs a) { mm2_body<13>(a); }
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
moearc_matmul2_q6_k_k(MatmulArgs a) { mm2_body<14>(a); }
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
moearc_matmul2_mxfp4_k(MatmulArgs a) { mm2_body<39>(a); }
