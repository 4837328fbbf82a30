// The reference's exact-arithmetic GEMM entry points on gfx950.
//
// gemm_naive (src/kernels/gemm.cl:26-51) and gemm_tiled (gemm.cl:74-136)
// compute, per output, acc = fma(A[row,k], B[k,col], acc) over k = 0..K-1 in
// fp32 from fp16 inputs and store RNE fp16.  Both kernels here keep that
// exact per-output fma sequence, so their results are bit-identical to each
// other and to a CPU restatement; only the work partition differs.
//   A [M,K], B [K,N], C [M,N], fp16 row-major.
#include "common.h"
#include "device_math.h"

namespace mvlm {

// One thread per output; threadIdx.x walks columns so B and C accesses are
// coalesced (the reference maps gid0 to rows, which strides B by N).
__global__ __launch_bounds__(256) void gemm_naive_kernel(const uint16_t* __restrict__ A,
                                                         const uint16_t* __restrict__ B,
                                                         uint16_t* __restrict__ C, int M, int N, int K) {
    int col = blockIdx.x * 16 + (threadIdx.x & 15);
    int row = blockIdx.y * 16 + (threadIdx.x >> 4);
    if (row >= M || col >= N) return;
    const uint16_t* a = A + (int64_t)row * K;
    const uint16_t* b = B + col;
    float acc = 0.0f;
    for (int k = 0; k < K; ++k)
        acc = __builtin_fmaf(f16_bits_to_f32(a[k]), f16_bits_to_f32(b[(int64_t)k * N]), acc);
    C[(int64_t)row * N + col] = f32_to_f16_bits(acc);
}

hipError_t launch_gemm_naive(hipStream_t s, const uint16_t* A, const uint16_t* B, uint16_t* C,
                             int M, int N, int K) {
    dim3 grid((N + 15) / 16, (M + 15) / 16);
    launch_kernel(gemm_naive_kernel, grid, dim3(256), 0, s, A, B, C, M, N, K);
    return hipGetLastError();
}

// 64x64 output tile per 256-thread block, 4x4 outputs per thread, K staged in
// 32-wide LDS slices (values widened to fp32 on the way in, which is exact).
// Each thread walks k in ascending order inside and across slices, so every
// output sees the same fma sequence as gemm_naive.
constexpr int TT = 64;    // tile edge
constexpr int TK = 32;    // K slice

__global__ __launch_bounds__(256) void gemm_tiled_kernel(const uint16_t* __restrict__ A,
                                                         const uint16_t* __restrict__ B,
                                                         uint16_t* __restrict__ C, int M, int N, int K) {
    __shared__ float As[TT][TK + 1];
    __shared__ float Bs[TK][TT];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int m0 = blockIdx.y * TT, n0 = blockIdx.x * TT;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;

    for (int k0 = 0; k0 < K; k0 += TK) {
        // A slice: 64 rows x 32 k; B slice: 32 k x 64 cols; 8 elements each per thread.
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            int idx = threadIdx.x + e * 256;
            int ar = idx / TK, ak = idx % TK;
            int gr = m0 + ar, gk = k0 + ak;
            As[ar][ak] = (gr < M && gk < K) ? f16_bits_to_f32(A[(int64_t)gr * K + gk]) : 0.0f;
            int bk = idx / TT, bc = idx % TT;
            int gk2 = k0 + bk, gc = n0 + bc;
            Bs[bk][bc] = (gk2 < K && gc < N) ? f16_bits_to_f32(B[(int64_t)gk2 * N + gc]) : 0.0f;
        }
        __syncthreads();
        const int kn = min(TK, K - k0);   // the zero padding beyond K is never accumulated
        for (int k = 0; k < kn; ++k) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[ty * 4 + i][k];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Bs[k][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int row = m0 + ty * 4 + i;
        if (row >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int col = n0 + tx * 4 + j;
            if (col < N) C[(int64_t)row * N + col] = f32_to_f16_bits(acc[i][j]);
        }
    }
}

hipError_t launch_gemm_tiled(hipStream_t s, const uint16_t* A, const uint16_t* B, uint16_t* C,
                             int M, int N, int K) {
    dim3 grid((N + TT - 1) / TT, (M + TT - 1) / TT);
    launch_kernel(gemm_tiled_kernel, grid, dim3(256), 0, s, A, B, C, M, N, K);
    return hipGetLastError();
}

}  // namespace mvlm
