// Element-wise kernels of the attention path: zero fill, f32 -> f16 narrowing and the paged KV
// append (one token, or a chunk of tokens). All are HBM-bound streaming kernels; each thread
// handles one element and the grids are sized on the host.
#include "common.h"

// Binary32 -> binary16 with the reference's rounding contract (kernels.cpp:152-186): IEEE
// round-to-nearest-even, subnormals rounded, overflow to +-inf. The hardware conversion
// (v_cvt_f16_f32 in the default RNE mode, f16 denormals preserved) implements exactly that; the
// one case it leaves open is a NaN's payload, which the reference defines as quiet bit | the top
// mantissa bits, so NaNs are encoded explicitly.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    const uint32_t x = __float_as_uint(f);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu) != 0u)
        return (uint16_t) (((x >> 16) & 0x8000u) | 0x7E00u | ((x & 0x7FFFFFu) >> 13));
    _Float16 h = (_Float16) f;
    return __builtin_bit_cast(uint16_t, h);
}

extern "C" __global__ void moearc_zero_k(float *dst, uint64_t n) {
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t) gridDim.x * blockDim.x)
        dst[i] = 0.0f;
}

extern "C" __global__ void moearc_quantize_f16_k(uint16_t *dst, const float *src, uint64_t n) {
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t) gridDim.x * blockDim.x)
        dst[i] = f32_to_f16_bits(src[i]);
}

// One token: element i of the [n_kv_heads][head_dim] row lands at base + i
// (layout [page][slot][kv_head][head_dim], kernels.cpp:1782-1799).
extern "C" __global__ void moearc_kv_append_k(void *k_pages, void *v_pages, const float *k,
                                              const float *v, uint64_t base, uint64_t row,
                                              uint32_t kv_type) {
    const uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= row) return;
    if (kv_type == MOEARC_KV_F16) {
        ((uint16_t *) k_pages)[base + i] = f32_to_f16_bits(k[i]);
        ((uint16_t *) v_pages)[base + i] = f32_to_f16_bits(v[i]);
    } else {
        ((float *) k_pages)[base + i] = k[i];
        ((float *) v_pages)[base + i] = v[i];
    }
}

// A chunk of tokens: token t goes to (page_ids[t], slots[t]). The host cannot see device-resident
// slots, so the bound is enforced here: a token whose slot lies outside the page is not written,
// and the refusal is recorded in *err (1), which the host reads back at its next synchronisation
// and reports as a failed call.
extern "C" __global__ void moearc_kv_append_chunk_k(void *k_pages, void *v_pages, const float *k,
                                                    const float *v, const uint32_t *page_ids,
                                                    const uint32_t *slots, uint64_t n_tok,
                                                    uint64_t row, uint64_t page_tokens,
                                                    uint32_t kv_type, uint32_t *err) {
    const uint64_t g = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_tok * row) return;
    const uint64_t t = g / row, i = g - t * row;
    const uint32_t slot = slots[t];
    if (slot >= page_tokens) {
        if (i == 0) *(volatile uint32_t *) err = 1u;  // every writer stores the same value
        return;
    }
    const uint64_t dst = ((uint64_t) page_ids[t] * page_tokens + slot) * row + i;
    if (kv_type == MOEARC_KV_F16) {
        ((uint16_t *) k_pages)[dst] = f32_to_f16_bits(k[g]);
        ((uint16_t *) v_pages)[dst] = f32_to_f16_bits(v[g]);
    } else {
        ((float *) k_pages)[dst] = k[g];
        ((float *) v_pages)[dst] = v[g];
    }
}

// Calibration read (moearc_read_floor): the HBM read rate a streaming kernel reaches on this device,
// for comparison with the attention kernels' traffic. Work-group g reads the 64 KiB at
// src + 64 KiB * g (16 KiB per wave: every load of a thread issued before any is used, 16 bytes per
// lane, consecutive lanes on consecutive 16-byte pieces) and writes the xor of its 32-bit words to
// out[g], so the loads cannot be dropped and the result can be checked.
#define MOEARC_READ_FLOOR_LOADS 16u
extern "C" __global__ void __launch_bounds__(256) moearc_read_floor_k(unsigned int *out, const u32x4_t *src,
                                                                      uint64_t n16) {
    __shared__ uint32_t part[4];
    const uint64_t base = (uint64_t) blockIdx.x * (256u * MOEARC_READ_FLOOR_LOADS) + threadIdx.x;
    u32x4_t v[MOEARC_READ_FLOOR_LOADS];
#pragma unroll
    for (uint32_t i = 0; i < MOEARC_READ_FLOOR_LOADS; ++i) {
        const uint64_t p = base + 256u * i;
        v[i] = p < n16 ? src[p] : (u32x4_t){0u, 0u, 0u, 0u};
    }
    uint32_t x = 0;
#pragma unroll
    for (uint32_t i = 0; i < MOEARC_READ_FLOOR_LOADS; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
#pragma unroll
    for (uint32_t m = 32; m >= 1; m >>= 1) x ^= (uint32_t) __shfl_xor((int) x, (int) m);
    if ((threadIdx.x & 63u) == 0) part[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// Calibration of the matrix cores (moearc_mfma_floor): the f16 MFMA rate this device sustains on
// data like the prefill's, for comparison with the prefill kernels. Each wave loads eight operand
// quads of f16 values (16 bytes per lane each) from src + 8 KiB * (global wave index) -- four A and
// four B operands of v_mfma_f32_32x32x16_f16 -- and runs four independent accumulator chains for
// `iters` rounds; in round i chain c multiplies A[(c + i) % 4] by B[(c + i) % 4], so every
// operand's bits keep entering the matrix core (its power, and with it the clock, depends on
// them). Two MFMAs per chain and round: 8 x 32,768 flops per wave and round. out[w] = the sum of
// wave w's 4 x 16 accumulators over its 64 lanes, which a host can recompute from src.
typedef float float16v_t __attribute__((ext_vector_type(16)));
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
moearc_mfma_floor_k(float *out, const u32x4_t *src, uint32_t iters) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t w = (uint64_t) blockIdx.x * 4u + (threadIdx.x >> 6);
    half8_t A[4], B[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        A[k] = __builtin_bit_cast(half8_t, src[w * 512u + 64u * k + lane]);
        B[k] = __builtin_bit_cast(half8_t, src[w * 512u + 64u * (4 + k) + lane]);
    }
    float16v_t D[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) D[c][i] = 0.f;
    for (uint32_t it = 0; it < iters; it += 4) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int k = (c + r) & 3;
                D[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[k], B[k], D[c], 0, 0, 0);
                D[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[k], B[k], D[c], 0, 0, 0);
            }
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int i = 0; i < 16; ++i) s += D[c][i];
#pragma unroll
    for (uint32_t m = 32; m >= 1; m >>= 1) s += __shfl_xor(s, (int) m);
    if (lane == 0) out[w] = s;
}
