// Row-wise argmax of logits on the device (the LM-head token pick).
//
// Replaces argmax_logits (src/models/moondream2.cpp:553-593), which reads the
// whole fp16 logit vector back to the host (100 KB for a 51200-token
// vocabulary) and scans it there.  Here one workgroup per row scans the row
// and writes only the winning index (4 bytes).
//
// Comparison key (the reference's fp16 decode, :571-583, extended to every
// dtype): zero-exponent values (zeros and subnormals) count as +0, all-ones
// exponents (inf and NaN) as +inf or -inf by their sign bit, everything else
// by value.  The smallest index wins among equal keys (the reference's strict
// '>' scan from index 0), so a row of all -inf (or -NaN) returns 0, as the
// reference does from its -1e30 start.
#include "common.h"
#include "device_math.h"

namespace mvlm {

template <int DT>
__device__ __forceinline__ float argmax_key(const void* row, int64_t i) {
    if constexpr (DT == MVLM_F32) {
        const uint32_t b = ((const uint32_t*)row)[i];
        const uint32_t e = (b >> 23) & 0xFFu;
        if (e == 0xFFu) return (b >> 31) ? -INFINITY : INFINITY;
        return e == 0 ? 0.0f : __uint_as_float(b);
    } else if constexpr (DT == MVLM_F16) {
        const uint16_t h = ((const uint16_t*)row)[i];
        const uint32_t e = (h >> 10) & 0x1Fu;
        if (e == 0x1Fu) return (h >> 15) ? -INFINITY : INFINITY;
        return e == 0 ? 0.0f : f16_bits_to_f32(h);
    } else {
        const uint16_t h = ((const uint16_t*)row)[i];
        const uint32_t e = (h >> 7) & 0xFFu;
        if (e == 0xFFu) return (h >> 15) ? -INFINITY : INFINITY;
        return e == 0 ? 0.0f : bf16_bits_to_f32(h);
    }
}

__device__ __forceinline__ bool argmax_better(float k, int i, float bk, int bi) {
    return k > bk || (k == bk && i < bi);
}

constexpr int ARGMAX_THREADS = 1024;

template <int DT>
__global__ __launch_bounds__(ARGMAX_THREADS) void argmax_kernel(const void* x, int n, int64_t ld, int* out) {
    __shared__ float wk[ARGMAX_THREADS / 64];
    __shared__ int wi[ARGMAX_THREADS / 64];
    const int es = DT == MVLM_F32 ? 4 : 2;
    const void* row = (const uint8_t*)x + (int64_t)blockIdx.x * ld * es;
    // each thread visits its indices in increasing order: strict '>' keeps the first
    float bk = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < n; i += ARGMAX_THREADS) {
        const float k = argmax_key<DT>(row, i);
        if (bi == 0x7FFFFFFF || k > bk) {
            bk = k;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ok = __shfl_xor(bk, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (argmax_better(ok, oi, bk, bi)) {
            bk = ok;
            bi = oi;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        wk[wave] = bk;
        wi[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < ARGMAX_THREADS / 64; ++w)
            if (argmax_better(wk[w], wi[w], bk, bi)) {
                bk = wk[w];
                bi = wi[w];
            }
        out[blockIdx.x] = bi;
    }
}

hipError_t launch_argmax(hipStream_t s, const void* x, int dtype, int rows, int n, int64_t ld, int* out) {
    const dim3 grid((unsigned)rows), block(ARGMAX_THREADS);
    switch (dtype) {
        case MVLM_F32: launch_kernel(argmax_kernel<MVLM_F32>, grid, block, 0, s, x, n, ld, out); break;
        case MVLM_F16: launch_kernel(argmax_kernel<MVLM_F16>, grid, block, 0, s, x, n, ld, out); break;
        case MVLM_BF16: launch_kernel(argmax_kernel<MVLM_BF16>, grid, block, 0, s, x, n, ld, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mvlm
