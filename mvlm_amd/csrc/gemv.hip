// Decode GEMV for dense packed weights: y[n] = sum_k x[k] * W[n][k].
//
// Replaces gemv (src/kernels/gemm.cl:215-270), which gives each 256-item
// work-group 4 outputs, strides k by 256 through an image and reduces through
// 8 LDS barrier steps.  Here one 64-lane wavefront owns R whole rows of the
// [N][K] weight: every lane streams 16 contiguous bytes per row per step
// (a wave reads 1 KiB of one row per load instruction, fully coalesced), the
// x segment it needs is loaded once and reused for all R rows, and the R
// partial sums are reduced across the wave with cross-lane shuffles, with no
// LDS and no barrier.  Weight rows are padded to ld (a multiple of 64) with
// zeros; x is read only below K.
#include "common.h"
#include "device_math.h"

namespace mvlm {

// Load E consecutive x values starting at k as fp32; zero beyond K.
template <typename XT, int E>
__device__ __forceinline__ void load_x(const XT* __restrict__ x, int k, int K, float (&out)[E]) {
    if (k + E <= K) {
        if constexpr (sizeof(XT) == 4) {
#pragma unroll
            for (int v = 0; v < E / 4; ++v) {
                float4 f = *reinterpret_cast<const float4*>(x + k + 4 * v);
                out[4 * v + 0] = f.x; out[4 * v + 1] = f.y; out[4 * v + 2] = f.z; out[4 * v + 3] = f.w;
            }
        } else if constexpr (E == 8) {
            u32x4 u = *reinterpret_cast<const u32x4*>(x + k);
            uint32_t w[4] = {u[0], u[1], u[2], u[3]};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                out[2 * v + 0] = bits_to_f32<XT>(((uint16_t)(w[v] & 0xFFFFu)));
                out[2 * v + 1] = bits_to_f32<XT>(((uint16_t)(w[v] >> 16)));
            }
        } else {  // 16-bit x with fp32 weights: 4 elements = 8 bytes
            u32x2 u = *reinterpret_cast<const u32x2*>(x + k);
            uint32_t w[2] = {u[0], u[1]};
#pragma unroll
            for (int v = 0; v < 2; ++v) {
                out[2 * v + 0] = bits_to_f32<XT>(((uint16_t)(w[v] & 0xFFFFu)));
                out[2 * v + 1] = bits_to_f32<XT>(((uint16_t)(w[v] >> 16)));
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) out[e] = (k + e < K) ? to_f32(x[k + e]) : 0.0f;
    }
}

// Widen the E weights held in one 16-byte load.
template <typename WT, int E>
__device__ __forceinline__ void widen_w(u32x4 u, float (&w)[E]) {
    uint32_t d[4] = {u[0], u[1], u[2], u[3]};
    if constexpr (sizeof(WT) == 4) {
#pragma unroll
        for (int v = 0; v < 4; ++v) w[v] = __uint_as_float(d[v]);
    } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            w[2 * v + 0] = bits_to_f32<WT>(((uint16_t)(d[v] & 0xFFFFu)));
            w[2 * v + 1] = bits_to_f32<WT>(((uint16_t)(d[v] >> 16)));
        }
    }
}

template <typename XT, typename WT, int R>
__global__ __launch_bounds__(256) void gemv_dense_kernel(const XT* __restrict__ x, const WT* __restrict__ W,
                                                         int64_t ld, void* __restrict__ y, int y_dtype,
                                                         int N, int K, const Epilogue ep) {
    constexpr int E = 16 / sizeof(WT);
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= N) return;
    const WT* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[r] = W + (int64_t)min(row0 + r, N - 1) * ld;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

#pragma unroll 2
    for (int k = lane * E; k < ld; k += 64 * E) {
        u32x4 wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[r] + k));
        float xv[E];
        load_x<XT, E>(x, k, K, xv);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float w[E];
            widen_w<WT, E>(wv[r], w);
#pragma unroll
            for (int e = 0; e < E; ++e) acc[r] = __builtin_fmaf(xv[e], w[e], acc[r]);
        }
    }
    // lane r < R ends with row r's sum and stores it
    const float tot = wave_sum_lanes<R>(acc, lane);
    const int row = row0 + (lane & (R - 1));
    if (lane < R && row < N) store_out(y, row, ep.any() ? apply_epilogue(ep, tot, row, row) : tot, y_dtype);
}

// Rows per wave: enough waves to cover the 256 CUs several times over, and
// up to 4 rows per wave on tall matrices so x is reused across rows.
static int rows_per_wave(int N) {
    if (N >= 8192) return 4;
    if (N >= 4096) return 2;
    return 1;
}

template <typename XT, typename WT>
static hipError_t launch_dense_xw(hipStream_t s, const void* x, const mvlm_weight* W, void* y, int y_dtype,
                                  int N, int K, const Epilogue& ep) {
    int R = rows_per_wave(N);
    unsigned grid = (unsigned)((N + 4 * R - 1) / (4 * R));
    const XT* xp = (const XT*)x;
    const WT* wp = (const WT*)W->data;
    switch (R) {
        case 4: launch_kernel(gemv_dense_kernel<XT, WT, 4>, dim3(grid), dim3(256), 0, s, xp, wp, W->ld, y, y_dtype, N, K, ep); break;
        case 2: launch_kernel(gemv_dense_kernel<XT, WT, 2>, dim3(grid), dim3(256), 0, s, xp, wp, W->ld, y, y_dtype, N, K, ep); break;
        default: launch_kernel(gemv_dense_kernel<XT, WT, 1>, dim3(grid), dim3(256), 0, s, xp, wp, W->ld, y, y_dtype, N, K, ep); break;
    }
    return hipGetLastError();
}

template <typename WT>
static hipError_t launch_dense_w(hipStream_t s, const void* x, int x_dtype, const mvlm_weight* W, void* y,
                                 int y_dtype, int N, int K, const Epilogue& ep) {
    switch (x_dtype) {
        case MVLM_F32: return launch_dense_xw<float, WT>(s, x, W, y, y_dtype, N, K, ep);
        case MVLM_F16: return launch_dense_xw<__half, WT>(s, x, W, y, y_dtype, N, K, ep);
        case MVLM_BF16: return launch_dense_xw<__hip_bfloat16, WT>(s, x, W, y, y_dtype, N, K, ep);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_dense(hipStream_t s, const void* x, int x_dtype, const mvlm_weight* W, void* y,
                             int y_dtype, int N, int K, const Epilogue* ep) {
    const Epilogue e = ep ? *ep : Epilogue{};
    switch (W->dtype) {
        case MVLM_F32: return launch_dense_w<float>(s, x, x_dtype, W, y, y_dtype, N, K, e);
        case MVLM_F16: return launch_dense_w<__half>(s, x, x_dtype, W, y, y_dtype, N, K, e);
        case MVLM_BF16: return launch_dense_w<__hip_bfloat16>(s, x, x_dtype, W, y, y_dtype, N, K, e);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mvlm
