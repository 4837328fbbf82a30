// Prefill / vision GEMM on CDNA4 matrix cores:
//   C[b][m][n] = sum_k A[b][m][k] * B[b][n][k]     (NT: both operands K-contiguous)
// A and B fp16 or bf16, fp32 accumulation, C stored fp32 / fp16 / bf16.
//
// This replaces gemm_image (src/kernels/gemm.cl:157-200) as the prefill path
// (dispatch_gemm_image, src/engine/compute.cpp:90-120; called for every
// projection in src/models/moondream2.cpp:374-508) and serves the batched
// attention scores Q*K^T (the dot in src/kernels/attention.cl:84-88).
//
// Structure: a 256-thread block (4 wavefronts, 2x2) owns a BM x BN tile of C.
// K advances in 32-wide slices: every thread fetches 16-byte chunks of the A
// and B slices into registers (the next slice is in flight while the current
// one is multiplied), writes them to LDS rows padded to 80 bytes (so the
// 16-byte fragment reads of 8 consecutive rows hit distinct banks), and each
// wave runs v_mfma_f32_32x32x16 on its (BM/2) x (BN/2) sub-tile.
// Operand layout of v_mfma_f32_32x32x16_{f16,bf16}: lane l supplies
// A[l%32][8*(l/32) .. +7] and B^T[l%32][8*(l/32) .. +7]; accumulator register
// r of lane l is C[8*(r/4) + 4*(l/32) + r%4][l%32].
#include "common.h"
#include "device_math.h"

namespace mvlm {

constexpr int BK = 32;
constexpr int LDS_STRIDE = BK + 8;   // elements per LDS row (80 bytes)

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <bool BF16, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                        void* __restrict__ C, int c_dtype, int M, int N, int K,
                                                        int64_t lda, int64_t ldb, int64_t ldc,
                                                        int64_t strideA, int64_t strideB, int64_t strideC) {
    constexpr int WM = BM / 2, WN = BN / 2;      // wave sub-tile
    constexpr int TM = WM / 32, TN = WN / 32;    // 32x32 MFMA tiles per wave
    constexpr int CA = BM / 64, CB = BN / 64;    // 16-byte chunks per thread per slice
    __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDS_STRIDE];

    const int bz = blockIdx.z;
    A += (int64_t)bz * strideA;
    B += (int64_t)bz * strideB;
    const int64_t c_off = (int64_t)bz * strideC;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    u32x4 ra[CA], rb[CB];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            int c = tid + i * 256, row = c >> 2, gk = k0 + (c & 3) * 8, gr = m0 + row;
            ra[i] = (gr < M && gk < K) ? *reinterpret_cast<const u32x4*>(A + (int64_t)gr * lda + gk) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            int c = tid + i * 256, row = c >> 2, gk = k0 + (c & 3) * 8, gn = n0 + row;
            rb[i] = (gn < N && gk < K) ? *reinterpret_cast<const u32x4*>(B + (int64_t)gn * ldb + gk) : u32x4{0, 0, 0, 0};
        }
    };
    auto lstore = [&]() {
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            int c = tid + i * 256;
            *reinterpret_cast<u32x4*>(&As[(c >> 2) * LDS_STRIDE + (c & 3) * 8]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < CB; ++i) {
            int c = tid + i * 256;
            *reinterpret_cast<u32x4*>(&Bs[(c >> 2) * LDS_STRIDE + (c & 3) * 8]) = rb[i];
        }
    };

    gload(0);
    for (int k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();
        lstore();
        __syncthreads();
        if (k0 + BK < K) gload(k0 + BK);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kof = ks * 16 + (lane >> 5) * 8;
            u32x4 a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                a[i] = *reinterpret_cast<const u32x4*>(&As[(wm * WM + i * 32 + (lane & 31)) * LDS_STRIDE + kof]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[j] = *reinterpret_cast<const u32x4*>(&Bs[(wn * WN + j * 32 + (lane & 31)) * LDS_STRIDE + kof]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<BF16>(a[i], b[j], acc[i][j]);
        }
    }

#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WN + j * 32 + (lane & 31);
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M) store_out(C, c_off + (int64_t)row * ldc + col, acc[i][j][r], c_dtype);
            }
        }
}

// Tile choice: the largest tile whose count fills the CUs in whole waves best.
struct TileCfg { int bm, bn; };

static TileCfg pick_tile(int M, int N, int batch, int num_cus) {
    const TileCfg cands[4] = {{128, 128}, {128, 64}, {64, 128}, {64, 64}};
    TileCfg best = cands[0];
    double best_eff = -1.0;
    for (const TileCfg& c : cands) {
        int64_t tiles = (int64_t)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * batch;
        int64_t rounds = (tiles + num_cus - 1) / num_cus;
        double eff = (double)tiles / (double)(rounds * num_cus);
        if (eff > best_eff + 0.05) { best_eff = eff; best = c; }
    }
    return best;
}

template <bool BF16>
static void launch_typed(hipStream_t s, TileCfg t, const uint16_t* A, const uint16_t* B, void* C, int c_dtype,
                         int batch, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
                         int64_t sA, int64_t sB, int64_t sC) {
    dim3 grid((N + t.bn - 1) / t.bn, (M + t.bm - 1) / t.bm, batch);
#define MVLM_LAUNCH(BMv, BNv)                                                                         \
    launch_kernel(gemm_mfma_kernel<BF16, BMv, BNv>, grid, dim3(256), 0, s, A, B, C, c_dtype, M, N, K, lda, \
                  ldb, ldc, sA, sB, sC)
    if (t.bm == 128 && t.bn == 128) MVLM_LAUNCH(128, 128);
    else if (t.bm == 128) MVLM_LAUNCH(128, 64);
    else if (t.bn == 128) MVLM_LAUNCH(64, 128);
    else MVLM_LAUNCH(64, 64);
#undef MVLM_LAUNCH
}

hipError_t launch_gemm_mfma(hipStream_t s, const void* A, int ab_dtype, const void* B, void* C, int c_dtype,
                            int batch, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
                            int64_t strideA, int64_t strideB, int64_t strideC, int num_cus) {
    TileCfg t = pick_tile(M, N, batch, num_cus > 0 ? num_cus : 256);
    if (ab_dtype == MVLM_BF16)
        launch_typed<true>(s, t, (const uint16_t*)A, (const uint16_t*)B, C, c_dtype, batch, M, N, K, lda, ldb, ldc,
                           strideA, strideB, strideC);
    else
        launch_typed<false>(s, t, (const uint16_t*)A, (const uint16_t*)B, C, c_dtype, batch, M, N, K, lda, ldb, ldc,
                            strideA, strideB, strideC);
    return hipGetLastError();
}

}  // namespace mvlm
