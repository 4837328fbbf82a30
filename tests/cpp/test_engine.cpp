// C++ tests of the mgpu:: drop-in (mvlm_amd/engine/mgpu_engine.h), in the
// manner of the reference's tests/test_device.cpp:22-244: every test needs a
// device and the program exits with 77 (skip) when init_device fails.
// Data are small integers, so every summation order gives the same bits and
// the expected outputs are computed exactly on the host.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "mgpu_engine.h"

static int g_failures = 0;
#define EXPECT_TRUE(c)                                                          \
    do {                                                                        \
        if (!(c)) { std::printf("  FAILED %s:%d: %s\n", __FILE__, __LINE__, #c); ++g_failures; } \
    } while (0)
#define EXPECT_EQ(a, b) EXPECT_TRUE((a) == (b))

using namespace mgpu;

static uint16_t h(float v) {      // exact for the small integers used here
    if (v == 0.0f) return 0;
    uint32_t u; std::memcpy(&u, &v, 4);
    uint32_t sign = (u >> 16) & 0x8000u, e = ((u >> 23) & 0xFF) - 127 + 15, m = (u >> 13) & 0x3FF;
    return (uint16_t)(sign | (e << 10) | m);
}
static float f(uint16_t x) {
    if ((x & 0x7FFF) == 0) return 0.0f;
    uint32_t sign = (x & 0x8000u) << 16, e = ((x >> 10) & 0x1F) - 15 + 127, m = (x & 0x3FF) << 13;
    uint32_t u = sign | (e << 23) | m; float v; std::memcpy(&v, &u, 4); return v;
}

static void test_buffer_pool(const DeviceInfo* dev) {
    std::printf("BufferPool\n");
    BufferPool pool;
    EXPECT_TRUE(init_buffer_pool(&pool, dev, 4096));
    Buffer a = get_current_buffer(&pool), b = get_next_buffer(&pool);
    EXPECT_TRUE(a && b && a != b);
    swap_buffers(&pool);
    EXPECT_EQ(get_current_buffer(&pool), b);
    EXPECT_EQ(get_next_buffer(&pool), a);
    destroy_buffer_pool(&pool);
    EXPECT_EQ(pool.size, (size_t)0);
}

static void test_gemm_variants(const DeviceInfo* dev) {
    std::printf("dispatch_gemm_naive / tiled / image and dispatch_gemv\n");
    const int M = 5, N = 37, K = 64;
    std::vector<uint16_t> A(M * K), B(K * N), C(M * N);
    std::vector<float> ref(M * N, 0.0f);
    for (int i = 0; i < M * K; ++i) A[i] = h((float)((i * 7) % 9 - 4));
    for (int i = 0; i < K * N; ++i) B[i] = h((float)((i * 5) % 7 - 3));
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n)
            for (int k = 0; k < K; ++k) ref[m * N + n] += f(A[m * K + k]) * f(B[k * N + n]);
    Buffer dA = create_buffer(dev, A.size() * 2, 0, A.data());
    Buffer dB = create_buffer(dev, B.size() * 2, 0, B.data());
    Buffer dC = create_buffer(dev, C.size() * 2);
    Weight W = create_weight_image(dev, K, N, B.data());
    EXPECT_TRUE(dA && dB && dC && W);
    const char* names[] = {"naive", "tiled", "image"};
    for (int v = 0; v < 3; ++v) {
        Event ev = v == 0 ? dispatch_gemm_naive(dev, nullptr, dA, dB, dC, M, N, K)
                 : v == 1 ? dispatch_gemm_tiled(dev, nullptr, dA, dB, dC, M, N, K)
                          : dispatch_gemm_image(dev, nullptr, dA, W, dC, M, N, K);
        EXPECT_TRUE(ev != nullptr);
        EXPECT_TRUE(wait_event(ev));
        EXPECT_TRUE(event_elapsed_ms(ev) >= 0.0);
        release_event(ev);
        EXPECT_TRUE(read_buffer(dev, dC, 0, C.size() * 2, C.data()));
        int bad = 0;
        for (int i = 0; i < M * N; ++i) bad += (f(C[i]) != ref[i]);
        if (bad) std::printf("  %s: %d mismatches\n", names[v], bad);
        EXPECT_EQ(bad, 0);
    }
    Buffer dy = create_buffer(dev, N * 2);
    Event ev = dispatch_gemv(dev, nullptr, dA, W, dy, N, K);   // x = row 0 of A
    EXPECT_TRUE(ev && wait_event(ev));
    release_event(ev);
    std::vector<uint16_t> y(N);
    EXPECT_TRUE(read_buffer(dev, dy, 0, N * 2, y.data()));
    for (int n = 0; n < N; ++n) EXPECT_EQ(f(y[n]), ref[n]);
    // the reference's failure contract: log and return nullptr
    std::printf("  (an error message is expected next)\n");
    EXPECT_TRUE(dispatch_gemm_naive(dev, nullptr, dA, dB, dC, M, N, 0) == nullptr);
    release_buffer(dA); release_buffer(dB); release_buffer(dC); release_buffer(dy); release_weight(W);
}

static void test_quant_gemv(const DeviceInfo* dev) {
    std::printf("dispatch_gemv_quant (Q8_0 and Q4_0 known-answer rows)\n");
    const int N = 3, K = 64;
    std::vector<uint8_t> q8(N * (K / 32) * 34), q4(N * (K / 32) * 18);
    std::vector<float> x(K), ref8(N, 0.0f), ref4(N, 0.0f);
    for (int k = 0; k < K; ++k) x[k] = (float)(k % 5 - 2);
    for (int n = 0; n < N; ++n)
        for (int b = 0; b < K / 32; ++b) {
            uint8_t* blk8 = &q8[(n * (K / 32) + b) * 34];
            uint8_t* blk4 = &q4[(n * (K / 32) + b) * 18];
            const uint16_t d8 = h(0.5f * (float)(n + 1)), d4 = h((float)(b + 1));
            std::memcpy(blk8, &d8, 2);
            std::memcpy(blk4, &d4, 2);
            for (int j = 0; j < 32; ++j) {
                const int q = (j * 3 + n) % 17 - 8;
                blk8[2 + j] = (uint8_t)(int8_t)q;
                ref8[n] += x[b * 32 + j] * (float)q * f(d8);
            }
            for (int j = 0; j < 16; ++j) {
                const int lo = (j + n) % 16, hi = (15 - j + b) % 16;
                blk4[2 + j] = (uint8_t)(lo | (hi << 4));
                ref4[n] += x[b * 32 + j] * (float)(lo - 8) * f(d4) + x[b * 32 + j + 16] * (float)(hi - 8) * f(d4);
            }
        }
    Buffer dx = create_buffer(dev, K * 4, 0, x.data());
    Buffer dy = create_buffer(dev, N * 4);
    for (int t = 0; t < 2; ++t) {
        Weight W = create_weight(dev, t == 0 ? MVLM_Q8_0 : MVLM_Q4_0, N, K, t == 0 ? (void*)q8.data() : (void*)q4.data());
        EXPECT_TRUE(W != nullptr);
        Event ev = dispatch_gemv_quant(dev, nullptr, dx, W, dy, 1, N, K);
        EXPECT_TRUE(ev && wait_event(ev));
        release_event(ev);
        std::vector<float> y(N);
        EXPECT_TRUE(read_buffer(dev, dy, 0, N * 4, y.data()));
        for (int n = 0; n < N; ++n) EXPECT_EQ(y[n], (t == 0 ? ref8 : ref4)[n]);
        release_weight(W);
    }
    release_buffer(dx); release_buffer(dy);
}

static void test_attention_and_token_pick(const DeviceInfo* dev) {
    std::printf("dispatch_attention_prefill / _decode and argmax_logits\n");
    // Q = 0 makes every visible score equal: the output is the mean of the
    // visible V rows (prefix means for the causal prefill, the full mean for
    // decode); small-integer V, fp16 output within half an ulp of the mean
    const int S = 8, H = 2, D = 64;
    std::vector<uint16_t> Q(S * H * D, 0), V(S * H * D), O(S * H * D);
    for (int i = 0; i < S * H * D; ++i) V[i] = h((float)((i * 7) % 11 - 5));
    Buffer dQ = create_buffer(dev, Q.size() * 2, 0, Q.data());
    Buffer dK = create_buffer(dev, V.size() * 2, 0, V.data());     // any finite keys
    Buffer dV = create_buffer(dev, V.size() * 2, 0, V.data());
    Buffer dO = create_buffer(dev, O.size() * 2);
    Event ev = dispatch_attention_prefill(dev, nullptr, dQ, dK, dV, dO, S, H, D);
    EXPECT_TRUE(ev && wait_event(ev));
    release_event(ev);
    EXPECT_TRUE(read_buffer(dev, dO, 0, O.size() * 2, O.data()));
    int bad = 0;
    for (int q = 0; q < S; ++q)
        for (int j = 0; j < H * D; ++j) {
            float sum = 0.0f;
            for (int k = 0; k <= q; ++k) sum += f(V[k * H * D + j]);
            const float want = sum / (float)(q + 1);
            bad += std::fabs(f(O[q * H * D + j]) - want) > std::fabs(want) * 1e-3f + 1e-6f;
        }
    EXPECT_EQ(bad, 0);
    ev = dispatch_attention_decode(dev, nullptr, dQ, dK, dV, dO, S, H, D);   // query = row 0 of Q
    EXPECT_TRUE(ev && wait_event(ev));
    release_event(ev);
    EXPECT_TRUE(read_buffer(dev, dO, 0, H * D * 2, O.data()));
    for (int j = 0; j < H * D; ++j) {
        float sum = 0.0f;
        for (int k = 0; k < S; ++k) sum += f(V[k * H * D + j]);
        EXPECT_TRUE(std::fabs(f(O[j]) - sum / S) <= std::fabs(sum / S) * 1e-3f + 1e-6f);
    }
    // token pick: the first of two equal maxima
    std::vector<uint16_t> logits(51200);
    for (int i = 0; i < 51200; ++i) logits[i] = h((float)(i % 97 - 60));
    logits[31000] = logits[40000] = h(100.0f);
    Buffer dl = create_buffer(dev, logits.size() * 2, 0, logits.data());
    EXPECT_EQ(argmax_logits(dev, dl, 51200), 31000);
    release_buffer(dQ); release_buffer(dK); release_buffer(dV); release_buffer(dO); release_buffer(dl);
}

int main() {
    DeviceInfo dev;
    if (!init_device(&dev)) {
        std::printf("SKIPPED: no device\n");
        return 77;
    }
    print_device_info(&dev);
    test_buffer_pool(&dev);
    test_gemm_variants(&dev);
    test_quant_gemv(&dev);
    test_attention_and_token_pick(&dev);
    EXPECT_TRUE(finish(&dev));
    destroy_device(&dev);
    std::printf(g_failures ? "FAILED (%d)\n" : "PASSED\n", g_failures);
    return g_failures ? 1 : 0;
}
