// General single-query paged attention: every shape the C ABI accepts (head_dim up to 1024, f32 or
// f16 KV, any page size, any GQA group), in f32 with an online softmax seeded by the sink.
//
// One work-group of 256 threads per (sequence, query head). Keys are taken 256 at a time: each
// thread scores one key (a serial dot product over head_dim against q staged in LDS), the chunk's
// max and sum are reduced across the work-group, and the P.V update is done with threads over the
// head's channels, so the V reads of one key are coalesced. This path exists for coverage of the
// reference's full argument space (its own tests use f32 KV, head_dim 128, page sizes 4 and 8);
// the gpt-oss shape runs the split-K MFMA kernel in decode_splitk.hip.
#include "common.h"

#define GEN_THREADS 256

__device__ __forceinline__ float kv_elem(const void *base, uint64_t i, uint32_t kv_type) {
    if (kv_type == MOEARC_KV_F16)
        return (float) __builtin_bit_cast(_Float16, ((const uint16_t *) base)[i]);
    return ((const float *) base)[i];
}

__device__ __forceinline__ float block_reduce_max(float x, float *red) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = x;
    __syncthreads();
    x = red[0];
    for (int i = 1; i < GEN_THREADS / 64; ++i) x = fmaxf(x, red[i]);
    return x;
}

__device__ __forceinline__ float block_reduce_sum(float x, float *red) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = x;
    __syncthreads();
    x = red[0];
    for (int i = 1; i < GEN_THREADS / 64; ++i) x += red[i];
    return x;
}

extern "C" __global__ __launch_bounds__(GEN_THREADS) void moearc_attn_decode_general_k(
    const DecodeGeneralArgs a) {
    __shared__ float q_s[1024];
    __shared__ float p_s[GEN_THREADS];
    __shared__ uint64_t row_s[GEN_THREADS];
    __shared__ float red[GEN_THREADS / 64];

    const uint32_t b = blockIdx.x / a.n_heads;
    const uint32_t h = blockIdx.x - b * a.n_heads;
    const uint32_t tid = threadIdx.x;
    const uint32_t D = a.head_dim;
    const uint32_t kvh = h / (a.n_heads / a.n_kv_heads);
    const uint64_t kv_row = (uint64_t) a.n_kv_heads * D;
    const uint32_t *bt = a.block_tables + (uint64_t) b * a.bt_stride;
    const uint32_t kb = a.kv_begin[b], ke = a.n_kv[b];

    const float *q = a.q + ((uint64_t) b * a.n_heads + h) * D;
    for (uint32_t d = tid; d < D; d += GEN_THREADS) q_s[d] = q[d];

    // Online softmax state, seeded with the sink: m = sink, l = e^0 = 1 (kernels.cpp:1877-1880).
    const bool have_sink = a.sinks != nullptr;
    float m = have_sink ? a.sinks[h] : -INFINITY;
    float l = have_sink ? 1.0f : 0.0f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // channels tid + 256*c

    for (uint32_t c0 = kb; c0 < ke; c0 += GEN_THREADS) {
        const uint32_t j = c0 + tid;
        const bool valid = j < ke;
        float s = -INFINITY;
        __syncthreads();  // q_s ready; previous chunk's p_s/row_s consumed
        if (valid) {
            const uint64_t row = (uint64_t) bt[j / a.page_tokens] * a.page_tokens + (j % a.page_tokens);
            const uint64_t base = row * kv_row + (uint64_t) kvh * D;
            row_s[tid] = base;
            float dot = 0.f;
            for (uint32_t d = 0; d < D; ++d) dot = fmaf(q_s[d], kv_elem(a.k_pages, base + d, a.kv_type), dot);
            s = dot * a.scale;
        }
        const float cmax = block_reduce_max(s, red);
        const float m_new = fmaxf(m, cmax);
        const float corr = expf(m - m_new);  // m = -inf on the first chunk without a sink: 0
        const float p = valid ? expf(s - m_new) : 0.f;
        p_s[tid] = p;
        const float psum = block_reduce_sum(p, red);  // contains the barrier that publishes p_s
        l = l * corr + psum;
        m = m_new;
        const uint32_t n_in = min(ke - c0, (uint32_t) GEN_THREADS);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t d = tid + c * GEN_THREADS;
            if (d >= D) break;
            float x = acc[c] * corr;
            for (uint32_t k = 0; k < n_in; ++k) x = fmaf(p_s[k], kv_elem(a.v_pages, row_s[k] + d, a.kv_type), x);
            acc[c] = x;
        }
    }

    const uint64_t o = ((uint64_t) b * a.n_heads + h) * D;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t d = tid + c * GEN_THREADS;
        if (d >= D) break;
        const float r = acc[c] / l;
        if (a.out_f16) ((_Float16 *) a.out)[o + d] = (_Float16) r;
        else ((float *) a.out)[o + d] = r;
    }
}
