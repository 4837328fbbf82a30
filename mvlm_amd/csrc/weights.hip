// Weight packing, exact dequantization and seeded synthetic inputs.
//
// GGUF block definitions (sizes pinned by the reference's
// tests/test_gguf.cpp:16-34 and src/models/gguf_loader.cpp:13-55):
//   Q8_0 block = { fp16 d; int8 qs[32] }   34 bytes, w_j = d * qs_j
//   Q4_0 block = { fp16 d; uint8 qs[16] }  18 bytes, w_j = ((qs_j & 15) - 8) * d,
//                                                      w_{j+16} = ((qs_j >> 4) - 8) * d
// The packed HBM layout splits codes and scales so that rows of codes are
// 16-byte aligned for 128-bit loads (GGUF's 34/18-byte blocks are not).
#include "common.h"
#include "device_math.h"

namespace mvlm {

// ---------------------------------------------------------------------------
// packing
// ---------------------------------------------------------------------------

// One thread per GGUF block: split {d, codes} into the scale and code arrays.
__global__ void pack_q8_0_kernel(const uint8_t* __restrict__ src, int8_t* __restrict__ codes,
                                 uint16_t* __restrict__ scales, int64_t nblocks) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* blk = src + b * 34;
    scales[b] = (uint16_t)(blk[0] | (blk[1] << 8));
    int8_t* dst = codes + b * 32;
#pragma unroll
    for (int j = 0; j < 32; ++j) dst[j] = (int8_t)blk[2 + j];
}

__global__ void pack_q4_0_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ codes,
                                 uint16_t* __restrict__ scales, int64_t nblocks) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint8_t* blk = src + b * 18;
    scales[b] = (uint16_t)(blk[0] | (blk[1] << 8));
    uint8_t* dst = codes + b * 16;
#pragma unroll
    for (int j = 0; j < 16; ++j) dst[j] = blk[2 + j];
}

// Dense, source [N][K]: copy each row into the [N][ld] layout, zero-padding
// columns K..ld-1.  T is the element bit container (uint32_t or uint16_t).
template <typename T>
__global__ void pack_dense_nk_kernel(const T* __restrict__ src, T* __restrict__ dst, int N, int K, int64_t ld) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t total = (int64_t)N * ld;
    if (i >= total) return;
    int64_t n = i / ld, k = i - n * ld;
    dst[i] = (k < K) ? src[n * K + k] : (T)0;
}

// Dense, source [K][N] (the reference's create_weight_image input): transpose
// through a 32x32 LDS tile so both reads and writes are coalesced.
template <typename T>
__global__ void pack_dense_kn_kernel(const T* __restrict__ src, T* __restrict__ dst, int N, int K, int64_t ld) {
    __shared__ T tile[32][33];
    int k0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
    int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 256 threads: 32 x 8
    for (int r = ty; r < 32; r += 8) {
        int k = k0 + r, n = n0 + tx;
        tile[r][tx] = (k < K && n < N) ? src[(int64_t)k * N + n] : (T)0;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8) {
        int n = n0 + r, k = k0 + tx;
        if (n < N && k < ld) dst[(int64_t)n * ld + k] = (k < K) ? tile[tx][r] : (T)0;
    }
}

hipError_t launch_pack(hipStream_t s, const void* src, int dtype, int layout, int N, int K, mvlm_weight* w) {
    const int threads = 256;
    if (dtype == MVLM_Q8_0 || dtype == MVLM_Q4_0) {
        int64_t nblocks = (int64_t)N * (K / 32);
        unsigned grid = (unsigned)((nblocks + threads - 1) / threads);
        if (dtype == MVLM_Q8_0)
            pack_q8_0_kernel<<<grid, threads, 0, s>>>((const uint8_t*)src, (int8_t*)w->data, (uint16_t*)w->scales, nblocks);
        else
            pack_q4_0_kernel<<<grid, threads, 0, s>>>((const uint8_t*)src, (uint8_t*)w->data, (uint16_t*)w->scales, nblocks);
        return hipGetLastError();
    }
    if (layout == MVLM_LAYOUT_NK) {
        int64_t total = (int64_t)N * w->ld;
        unsigned grid = (unsigned)((total + threads - 1) / threads);
        if (dtype == MVLM_F32)
            pack_dense_nk_kernel<uint32_t><<<grid, threads, 0, s>>>((const uint32_t*)src, (uint32_t*)w->data, N, K, w->ld);
        else
            pack_dense_nk_kernel<uint16_t><<<grid, threads, 0, s>>>((const uint16_t*)src, (uint16_t*)w->data, N, K, w->ld);
    } else {
        dim3 grid((unsigned)((w->ld + 31) / 32), (unsigned)((N + 31) / 32));
        if (dtype == MVLM_F32)
            pack_dense_kn_kernel<uint32_t><<<grid, threads, 0, s>>>((const uint32_t*)src, (uint32_t*)w->data, N, K, w->ld);
        else
            pack_dense_kn_kernel<uint16_t><<<grid, threads, 0, s>>>((const uint16_t*)src, (uint16_t*)w->data, N, K, w->ld);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// exact dequantization to fp32 [N][K]
// ---------------------------------------------------------------------------

__global__ void dequant_q8_0_kernel(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
                                    float* __restrict__ out, int64_t total) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    out[i] = q8_value(codes[i], f16_bits_to_f32(scales[i >> 5]));
}

__global__ void dequant_q4_0_kernel(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
                                    float* __restrict__ out, int64_t total) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    int64_t b = i >> 5;
    int j = (int)(i & 31);
    uint8_t byte = codes[b * 16 + (j & 15)];
    int code = (j < 16) ? (byte & 15) : (byte >> 4);
    out[i] = q4_value(code, f16_bits_to_f32(scales[b]));
}

template <typename T>
__global__ void dequant_dense_kernel(const T* __restrict__ data, float* __restrict__ out, int N, int K, int64_t ld) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)N * K) return;
    int64_t n = i / K, k = i - n * K;
    out[i] = to_f32(data[n * ld + k]);
}

hipError_t launch_dequant(hipStream_t s, const mvlm_weight* w, float* out) {
    const int threads = 256;
    int64_t total = (int64_t)w->N * w->K;
    unsigned grid = (unsigned)((total + threads - 1) / threads);
    switch (w->dtype) {
        case MVLM_Q8_0:
            dequant_q8_0_kernel<<<grid, threads, 0, s>>>((const int8_t*)w->data, (const uint16_t*)w->scales, out, total);
            break;
        case MVLM_Q4_0:
            dequant_q4_0_kernel<<<grid, threads, 0, s>>>((const uint8_t*)w->data, (const uint16_t*)w->scales, out, total);
            break;
        case MVLM_F32:
            dequant_dense_kernel<float><<<grid, threads, 0, s>>>((const float*)w->data, out, w->N, w->K, w->ld);
            break;
        case MVLM_F16:
            dequant_dense_kernel<__half><<<grid, threads, 0, s>>>((const __half*)w->data, out, w->N, w->K, w->ld);
            break;
        case MVLM_BF16:
            dequant_dense_kernel<__hip_bfloat16><<<grid, threads, 0, s>>>((const __hip_bfloat16*)w->data, out, w->N, w->K, w->ld);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// seeded synthetic inputs (SplitMix64 at a counter, Box-Muller in fp64)
// ---------------------------------------------------------------------------

__device__ inline uint64_t splitmix64_at(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1u) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ inline double uniform_at(uint64_t seed, uint64_t index) {
    return (double)((splitmix64_at(seed, index) >> 11) + 1u) * 0x1.0p-53;
}

__device__ inline double normal_at(uint64_t seed, uint64_t index) {
    uint64_t j = index >> 1;
    double u1 = uniform_at(seed, 2 * j), u2 = uniform_at(seed, 2 * j + 1);
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586476925286766559 * u2;
    return (index & 1u) ? r * sin(t) : r * cos(t);
}

__global__ void fill_normal_kernel(void* dst, int dtype, int64_t count, uint64_t seed, double sd) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    float v = (float)(sd * normal_at(seed, (uint64_t)i));
    if (dtype == MVLM_F32) ((float*)dst)[i] = v;
    else if (dtype == MVLM_F16) ((uint16_t*)dst)[i] = f32_to_f16_bits(v);
    else ((uint16_t*)dst)[i] = f32_to_bf16_bits(v);
}

#define CODE_STREAM 0x5157ull

__global__ void random_q8_0_kernel(int8_t* __restrict__ codes, uint16_t* __restrict__ scales,
                                   int64_t nblocks, uint64_t seed, double wstd) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    scales[b] = f32_to_f16_bits((float)(fabs(wstd * normal_at(seed, (uint64_t)b)) / 127.0));
    int8_t* dst = codes + b * 32;
#pragma unroll 4
    for (int j = 0; j < 32; ++j)
        dst[j] = (int8_t)((int)(splitmix64_at(seed ^ CODE_STREAM, (uint64_t)b * 32 + j) % 255u) - 127);
}

__global__ void random_q4_0_kernel(uint8_t* __restrict__ codes, uint16_t* __restrict__ scales,
                                   int64_t nblocks, uint64_t seed, double wstd) {
    int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    scales[b] = f32_to_f16_bits((float)(fabs(wstd * normal_at(seed, (uint64_t)b)) / 8.0));
    uint8_t* dst = codes + b * 16;
#pragma unroll 4
    for (int j = 0; j < 16; ++j) {
        uint32_t lo = (uint32_t)(splitmix64_at(seed ^ CODE_STREAM, (uint64_t)b * 32 + j) & 15u);
        uint32_t hi = (uint32_t)(splitmix64_at(seed ^ CODE_STREAM, (uint64_t)b * 32 + j + 16) & 15u);
        dst[j] = (uint8_t)(lo | (hi << 4));
    }
}

__global__ void random_dense_kernel(void* __restrict__ data, int N, int K, int64_t ld, uint64_t seed, double sd, int dtype) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)N * ld) return;
    int64_t n = i / ld, k = i - n * ld;
    float v = (k < K) ? (float)(sd * normal_at(seed, (uint64_t)(n * K + k))) : 0.0f;
    if (dtype == MVLM_F32) ((float*)data)[i] = v;
    else if (dtype == MVLM_F16) ((uint16_t*)data)[i] = f32_to_f16_bits(v);
    else ((uint16_t*)data)[i] = f32_to_bf16_bits(v);
}

hipError_t launch_fill_normal(hipStream_t s, void* dst, int dtype, size_t count, uint64_t seed, double sd) {
    const int threads = 256;
    unsigned grid = (unsigned)((count + threads - 1) / threads);
    fill_normal_kernel<<<grid, threads, 0, s>>>(dst, dtype, (int64_t)count, seed, sd);
    return hipGetLastError();
}

hipError_t launch_weight_random(hipStream_t s, mvlm_weight* w, uint64_t seed, double wstd) {
    const int threads = 256;
    if (w->dtype == MVLM_Q8_0 || w->dtype == MVLM_Q4_0) {
        int64_t nblocks = (int64_t)w->N * (w->K / 32);
        unsigned grid = (unsigned)((nblocks + threads - 1) / threads);
        if (w->dtype == MVLM_Q8_0)
            random_q8_0_kernel<<<grid, threads, 0, s>>>((int8_t*)w->data, (uint16_t*)w->scales, nblocks, seed, wstd);
        else
            random_q4_0_kernel<<<grid, threads, 0, s>>>((uint8_t*)w->data, (uint16_t*)w->scales, nblocks, seed, wstd);
        return hipGetLastError();
    }
    int64_t total = (int64_t)w->N * w->ld;
    unsigned grid = (unsigned)((total + threads - 1) / threads);
    random_dense_kernel<<<grid, threads, 0, s>>>(w->data, w->N, w->K, w->ld, seed, wstd, w->dtype);
    return hipGetLastError();
}

}  // namespace mvlm
