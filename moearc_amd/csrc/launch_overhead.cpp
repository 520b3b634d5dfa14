// What one launch costs, apart from what the kernel computes: the measurement of
// crates/moearc-kernels/examples/launch_overhead.rs:21-125, through this library's C ABI.
//
//   submit only          moearc_add over one element, REPS submissions, then one wait
//   submit + wait        the same with a moearc_sync after every submission
//   4-byte device->host  moearc_copy_d2h of one float
//   attn_decode submit   moearc_attn_decode at the gpt-oss shape (64 q heads, 8 KV heads, head_dim
//                        64, 64-token pages) with n_kv = 1: f32 KV as the reference's example runs it
//                        (the general kernel here), and f16 KV (the split-K kernel)
//
// Prints one JSON object (microseconds per operation). Built beside libmoearc_attn.so by
// moearc_amd/build.py; bench.py runs it.
#include "moearc_attn.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

namespace {

constexpr int REPS = 2000;

void check(int rc, const char *what) {
    if (rc != 0) {
        std::fprintf(stderr, "launch_overhead: %s returned %d\n", what, rc);
        std::exit(1);
    }
}

template <typename F>
double per_op_us(moearc_ctx *c, F &&f, bool sync_after) {
    for (int i = 0; i < 64; ++i) f();  // warm-up: first submissions build queues and load modules
    check(moearc_sync(c), "sync");
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < REPS; ++i) {
        f();
        if (sync_after) check(moearc_sync(c), "sync");
    }
    check(moearc_sync(c), "sync");
    const auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double, std::micro>(t1 - t0).count() / REPS;
}

}  // namespace

int main() {
    moearc_ctx *c = moearc_ctx_create();
    if (!c) {
        std::fprintf(stderr, "launch_overhead: no device\n");
        return 1;
    }
    char name[256] = {0};
    check(moearc_device_name(c, name, sizeof(name)), "device_name");

    auto alloc = [&](unsigned long bytes) {
        void *p = moearc_alloc_device(c, bytes);
        if (!p) {
            std::fprintf(stderr, "launch_overhead: allocation of %lu bytes failed\n", bytes);
            std::exit(1);
        }
        return p;
    };
    float *a = (float *) alloc(1024 * 4), *b = (float *) alloc(1024 * 4), *out = (float *) alloc(1024 * 4);
    std::vector<float> ones(1024, 1.0f), twos(1024, 2.0f);
    check(moearc_copy_h2d(c, a, ones.data(), 1024 * 4), "copy_h2d");
    check(moearc_copy_h2d(c, b, twos.data(), 1024 * 4), "copy_h2d");

    auto add1 = [&] { check(moearc_add(c, out, a, b, 1), "add"); };
    const double submit = per_op_us(c, add1, false);
    const double submit_wait = per_op_us(c, add1, true);
    float host = 0.f;
    const double readback = per_op_us(c, [&] { check(moearc_copy_d2h(c, &host, out, 4), "copy_d2h"); }, false);

    // attention at the north-star shape, one key
    const unsigned long H = 64, G = 8, D = 64, PT = 64;
    const unsigned long pool = PT * G * D;
    void *k32 = alloc(pool * 4), *v32 = alloc(pool * 4), *k16 = alloc(pool * 2), *v16 = alloc(pool * 2);
    float *q = (float *) alloc(H * D * 4), *attn = (float *) alloc(H * D * 4);
    unsigned int *bt = (unsigned int *) alloc(4);
    std::vector<float> zeros(pool, 0.0f);
    const unsigned int page0 = 0;
    check(moearc_copy_h2d(c, k32, zeros.data(), pool * 4), "copy_h2d");
    check(moearc_copy_h2d(c, v32, zeros.data(), pool * 4), "copy_h2d");
    check(moearc_copy_h2d(c, k16, zeros.data(), pool * 2), "copy_h2d");
    check(moearc_copy_h2d(c, v16, zeros.data(), pool * 2), "copy_h2d");
    check(moearc_copy_h2d(c, q, zeros.data(), H * D * 4), "copy_h2d");
    check(moearc_copy_h2d(c, bt, &page0, 4), "copy_h2d");
    const double attn_f32 = per_op_us(c, [&] {
        check(moearc_attn_decode(c, attn, q, k32, v32, bt, nullptr, H, G, D, 0, 1, PT, 0.125f, 0), "attn_decode");
    }, false);
    const double attn_f16 = per_op_us(c, [&] {
        check(moearc_attn_decode(c, attn, q, k16, v16, bt, nullptr, H, G, D, 0, 1, PT, 0.125f, 1), "attn_decode");
    }, false);

    std::printf("{\"device\": \"%s\", \"reps\": %d, \"submit_only_us\": %.3f, \"submit_wait_us\": %.3f, "
                "\"readback_4b_us\": %.3f, \"attn_decode_submit_us_f32kv\": %.3f, "
                "\"attn_decode_submit_us_f16kv\": %.3f, \"sync_cost_us\": %.3f}\n",
                name, REPS, submit, submit_wait, readback, attn_f32, attn_f16, submit_wait - submit);
    for (void *p : {(void *) a, (void *) b, (void *) out, k32, v32, k16, v16, (void *) q, (void *) attn, (void *) bt})
        moearc_free_device(c, p);
    moearc_ctx_destroy(c);
    return 0;
}
