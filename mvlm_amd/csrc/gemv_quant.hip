// Dequantizing GEMV / skinny GEMM over GGUF Q8_0 and Q4_0 weights:
// Y[m][n] = sum_k X[m][k] * w(n, k), 1 <= M <= 16, X and Y fp32.
//
// The reference plans this kernel (README.md:57, PLAN.md:65) but never wrote
// it.  Weights stream once from HBM in the packed split layout (codes rows
// 16-byte aligned, fp16 scales in their own array).  One wavefront owns R
// rows; per step each lane takes one 16-byte code vector per row:
//   Q8_0: 16 codes = half a block (a wave covers 1024 weights of a row),
//   Q4_0: 32 codes = one block   (a wave covers 2048 weights of a row).
// Codes become fp32 in registers (v_cvt_f32_i32 with a byte select for
// int8, v_cvt_f32_ubyte* on masked nibbles), the block sum
// s = sum_j x_j * q_j is formed with fp32 fma, and the block scale is applied
// once per block: acc += d * s  (Q4_0: acc += d * (s - 8 * sum_j x_j)).
// Factoring d out of the block changes rounding only within the fp32
// tolerance; the exact per-weight values d*q are what mvlm_weight_dequant
// produces.  Partial sums are reduced across the wave with shuffles.
#include "common.h"
#include "device_math.h"

namespace mvlm {

__device__ __forceinline__ void load_f32x16(const float* __restrict__ p, float (&v)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f32x4 f = *reinterpret_cast<const f32x4*>(p + 4 * i);
        v[4 * i + 0] = f[0]; v[4 * i + 1] = f[1]; v[4 * i + 2] = f[2]; v[4 * i + 3] = f[3];
    }
}

template <int R, int MT>
__global__ __launch_bounds__(256) void gemv_q8_0_kernel(const float* __restrict__ X, const int8_t* __restrict__ codes,
                                                        const uint16_t* __restrict__ scales, float* __restrict__ Y,
                                                        int M, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= N) return;
    const int nb = K >> 5;
    int row[R];
#pragma unroll
    for (int r = 0; r < R; ++r) row[r] = min(row0 + r, N - 1);
    float acc[MT][R];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    for (int k = lane * 16; k < K; k += 1024) {
        u32x4 q[R];
        float d[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            q[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + (int64_t)row[r] * K + k));
            d[r] = f16_bits_to_f32(scales[(int64_t)row[r] * nb + (k >> 5)]);
        }
        float w[R][16];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < 16; ++j) w[r][j] = (float)(int8_t)(q[r][j >> 2] >> (8 * (j & 3)));
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m < M) {
                float xv[16];
                load_f32x16(X + (int64_t)m * K + k, xv);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float s = 0.0f;
#pragma unroll
                    for (int j = 0; j < 16; ++j) s = __builtin_fmaf(xv[j], w[r][j], s);
                    acc[m][r] = __builtin_fmaf(d[r], s, acc[m][r]);
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m >= M) continue;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = wave_sum(acc[m][r]);
            if (lane == 0 && row0 + r < N) Y[(int64_t)m * N + row0 + r] = v;
        }
    }
}

template <int R, int MT>
__global__ __launch_bounds__(256) void gemv_q4_0_kernel(const float* __restrict__ X, const uint8_t* __restrict__ codes,
                                                        const uint16_t* __restrict__ scales, float* __restrict__ Y,
                                                        int M, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= N) return;
    const int nb = K >> 5;
    int row[R];
#pragma unroll
    for (int r = 0; r < R; ++r) row[r] = min(row0 + r, N - 1);
    float acc[MT][R];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

    for (int b = lane; b < nb; b += 64) {
        const int k = b << 5;
        u32x4 q[R];
        float d[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            q[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes + (int64_t)row[r] * (K >> 1) + (b << 4)));
            d[r] = f16_bits_to_f32(scales[(int64_t)row[r] * nb + b]);
        }
        // code of weight j (0..15) is the low nibble of byte j, of weight j+16 the high nibble
        float w[R][32];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t lo = nibbles_to_bytes(q[r][i]);
                const uint32_t hi = nibbles_to_bytes(q[r][i] >> 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w[r][4 * i + e] = (float)((lo >> (8 * e)) & 0xFFu);
                    w[r][16 + 4 * i + e] = (float)((hi >> (8 * e)) & 0xFFu);
                }
            }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            if (m >= M) continue;
            float xv[32];
            const float* xp = X + (int64_t)m * K + k;
            float lo16[16], hi16[16];
            load_f32x16(xp, lo16);
            load_f32x16(xp + 16, hi16);
            float sx = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) { xv[j] = lo16[j]; xv[16 + j] = hi16[j]; }
#pragma unroll
            for (int j = 0; j < 32; ++j) sx += xv[j];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < 32; ++j) s = __builtin_fmaf(xv[j], w[r][j], s);
                acc[m][r] = __builtin_fmaf(d[r], __builtin_fmaf(-8.0f, sx, s), acc[m][r]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        if (m >= M) continue;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float v = wave_sum(acc[m][r]);
            if (lane == 0 && row0 + r < N) Y[(int64_t)m * N + row0 + r] = v;
        }
    }
}

template <int R, int MT>
static void launch_q(hipStream_t s, const float* X, const mvlm_weight* W, float* Y, int M, int N, int K) {
    unsigned grid = (unsigned)((N + 4 * R - 1) / (4 * R));
    if (W->dtype == MVLM_Q8_0)
        launch_kernel(gemv_q8_0_kernel<R, MT>, dim3(grid), dim3(256), 0, s, X, (const int8_t*)W->data,
                      (const uint16_t*)W->scales, Y, M, N, K);
    else
        launch_kernel(gemv_q4_0_kernel<R, MT>, dim3(grid), dim3(256), 0, s, X, (const uint8_t*)W->data,
                      (const uint16_t*)W->scales, Y, M, N, K);
}

hipError_t launch_gemv_quant(hipStream_t s, const float* X, const mvlm_weight* W, float* Y, int M, int N, int K) {
    if (M <= 1) {
        if (N >= 8192) launch_q<4, 1>(s, X, W, Y, M, N, K);
        else if (N >= 4096) launch_q<2, 1>(s, X, W, Y, M, N, K);
        else launch_q<1, 1>(s, X, W, Y, M, N, K);
    } else if (M <= 2) {
        launch_q<2, 2>(s, X, W, Y, M, N, K);
    } else if (M <= 4) {
        launch_q<2, 4>(s, X, W, Y, M, N, K);
    } else if (M <= 8) {
        launch_q<1, 8>(s, X, W, Y, M, N, K);
    } else {
        launch_q<1, 16>(s, X, W, Y, M, N, K);
    }
    return hipGetLastError();
}

}  // namespace mvlm
