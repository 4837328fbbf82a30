// The reference's exact-arithmetic GEMM entry points on gfx950.
//
// gemm_naive (src/kernels/gemm.cl:26-51) and gemm_tiled (gemm.cl:74-136)
// compute, per output, acc = fma(A[row,k], B[k,col], acc) over k = 0..K-1 in
// fp32 from fp16 inputs and store RNE fp16.  Both kernels here keep that
// exact per-output fma sequence, so their results are bit-identical to each
// other and to a CPU restatement; only the work partition differs.
//   A [M,K], B [K,N], C [M,N], fp16 row-major.
// gemv_exact keeps the reference gemv's split of K over 256 partial sums and
// its fold order on the packed fp16 weight.
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

// gemv (gemm.cl:215-270) as launched by dispatch_gemv (compute.cpp:141-147):
// y[n] = sum_k x[k] W[n,k] with the reference's summation order.  There, one
// 256-item group owns 4 outputs; item L keeps p = fma(x[k], W[n,k], p) over
// k = L, L+256, L+512, ... and the 256 partials are then folded by
// red[L] = red[L] + red[L+s] for s = 128, 64, ..., 1.
//
// Here one wave owns GX_ROWS outputs of the packed [N][ld] fp16 weight (rows
// zero padded to ld = K rounded up to 64, 128-byte aligned) and streams
// them: lane l holds the partials L = 4l + c, c = 0..3, and in the window
// starting at k0 reads W[n, k0+4l .. k0+4l+3] and the same x quad, one 8-byte
// load each, so a wave's loads are 512 contiguous bytes per row and every
// partial sees the reference's fma sequence.  GX_WIN windows are loaded
// before any is used.  The fold keeps the reference's pairs: strides 128..4
// pair lane l with lane l + s/4 (lane shuffles), strides 2 and 1 pair the
// four partials of lane 0.  Those pairs fix every rounding, so y is
// bit-identical to the reference's.
constexpr int GX_ROWS = 2;   // outputs per wave
constexpr int GX_WIN = 8;    // 256-wide k windows loaded together

template <int WIN>
__device__ __forceinline__ void gemv_exact_windows(const uint16_t* __restrict__ x, const uint16_t* const* rows,
                                                   int k0, int lane, float (&p)[GX_ROWS][4]) {
    uint2 w[WIN][GX_ROWS], xq[WIN];
#pragma unroll
    for (int v = 0; v < WIN; ++v) {
        const int k = k0 + 256 * v + 4 * lane;
        xq[v] = *reinterpret_cast<const uint2*>(x + k);
#pragma unroll
        for (int r = 0; r < GX_ROWS; ++r) w[v][r] = *reinterpret_cast<const uint2*>(rows[r] + k);
    }
    __builtin_amdgcn_sched_barrier(0);   // every load of the windows is issued before the first use
#pragma unroll
    for (int v = 0; v < WIN; ++v) {
        const float xf[4] = {f16_bits_to_f32(xq[v].x & 0xFFFF), f16_bits_to_f32(xq[v].x >> 16),
                             f16_bits_to_f32(xq[v].y & 0xFFFF), f16_bits_to_f32(xq[v].y >> 16)};
#pragma unroll
        for (int r = 0; r < GX_ROWS; ++r) {
            const float wf[4] = {f16_bits_to_f32(w[v][r].x & 0xFFFF), f16_bits_to_f32(w[v][r].x >> 16),
                                 f16_bits_to_f32(w[v][r].y & 0xFFFF), f16_bits_to_f32(w[v][r].y >> 16)};
#pragma unroll
            for (int c = 0; c < 4; ++c) p[r][c] = __builtin_fmaf(xf[c], wf[c], p[r][c]);
        }
    }
}

__global__ __launch_bounds__(256) void gemv_exact_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ W, int64_t ld,
                                                         uint16_t* __restrict__ y, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * GX_ROWS;
    if (n0 >= N) return;   // no block-wide barrier follows
    const uint16_t* rows[GX_ROWS];
#pragma unroll
    for (int r = 0; r < GX_ROWS; ++r) rows[r] = W + (int64_t)min(n0 + r, N - 1) * ld;
    float p[GX_ROWS][4];
#pragma unroll
    for (int r = 0; r < GX_ROWS; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) p[r][c] = 0.0f;
    int k0 = 0;
    for (; k0 + 256 * GX_WIN <= K; k0 += 256 * GX_WIN) gemv_exact_windows<GX_WIN>(x, rows, k0, lane, p);
    for (; k0 + 256 <= K; k0 += 256) gemv_exact_windows<1>(x, rows, k0, lane, p);
    if (k0 < K) {   // the last, partial window: element loads below K only
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int k = k0 + 4 * lane + c;
            if (k < K) {
                const float xv = f16_bits_to_f32(x[k]);
#pragma unroll
                for (int r = 0; r < GX_ROWS; ++r)
                    p[r][c] = __builtin_fmaf(xv, f16_bits_to_f32(rows[r][k]), p[r][c]);
            }
        }
    }
    // lane l < d receives the partial of lane l + d: d = 32 .. 1 are the strides 128 .. 4
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1)
#pragma unroll
        for (int r = 0; r < GX_ROWS; ++r)
#pragma unroll
            for (int c = 0; c < 4; ++c) p[r][c] = p[r][c] + __shfl_down(p[r][c], d, 64);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < GX_ROWS; ++r)
            if (n0 + r < N) y[n0 + r] = f32_to_f16_bits((p[r][0] + p[r][2]) + (p[r][1] + p[r][3]));
    }
}

hipError_t launch_gemv_exact(hipStream_t s, const uint16_t* x, const mvlm_weight* W, uint16_t* y) {
    const int per_block = 4 * GX_ROWS;
    dim3 grid((W->N + per_block - 1) / per_block);
    launch_kernel(gemv_exact_kernel, grid, dim3(256), 0, s, x, (const uint16_t*)W->data, (int64_t)W->ld, y,
                  W->N, W->K);
    return hipGetLastError();
}

}  // namespace mvlm
