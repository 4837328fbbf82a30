// Batched NT products with a short inner dimension and a dense fp32 C:
//   C[b][m][n] = sum_k A[b][m][k] * B[b][n][k],  K <= 128, ldc == N,
// the attention scores Q * K^T of SigLIP (16 heads x [729 x 72] * [72 x 729],
// the dot of src/kernels/attention.cl:84-88) and any product shaped like it.
//
// Such a product moves little data in (Q and K: 3.4 MB) and much out (fp32
// scores: 34 MB), so it is bound by HBM writes.  With N = 729 a C row is 2916
// bytes and starts 4-byte aligned, so a tiled GEMM that writes row pieces of a
// tile issues partial 64-byte writes at every piece's edges (the general MFMA
// GEMM wrote 1.4x the score bytes here).  Here the C rows of one batch are
// cut into blocks of 16 consecutive rows; a block's part of C is one
// contiguous range of 16 N floats, computed on the matrix cores into LDS and
// then streamed out with 16-byte stores aligned in HBM (the LDS copy is shifted
// by the range's start modulo 4 floats, so aligned global chunks come from
// aligned LDS chunks; at most 3 + 3 floats at the ends use 4-byte stores).
//
// A workgroup serves one batch and the row blocks p, p + P, p + 2P, ...  Its
// 8 waves split the columns (16-column blocks dealt in turn, at most 8 per
// wave) and load the B fragments of their columns into registers once, for
// every row block they compute: B (K of attention) is read from L2 once per
// workgroup instead of once per row block.  The A rows of all its row blocks
// are staged into LDS first, so the row-block loop issues no vector loads and
// never waits on the vector-memory counter: the stores of every block stay in
// flight while the next blocks are computed (loads and stores share that
// counter, so a wait for a load would also wait for them).
//
// Products: v_mfma_f32_16x16x32_{f16,bf16}.  Operand layout: lane l supplies
// A[l%16][8*(l/16) .. +7] and B^T[l%16][8*(l/16) .. +7] for k-step ks (K
// offset 32 ks); accumulator register i of lane l is C[4*(l/16) + i][l%16].
// K is a multiple of 8: an 8-element group is inside K or past it, and groups
// past K are zero in registers (never loaded: B's groups past K may lie past
// its buffer).  Rows of A past M load row M - 1 and columns of B past N load
// column N - 1; their products are never stored.  fp16/bf16 products are exact
// in fp32; the matrix core's accumulation order differs from an fma chain in
// ascending k, within the 1e-3 relative bound of 16-bit inputs.
#include "common.h"
#include "device_math.h"

#include <cstdlib>

namespace mvlm {

struct SmallKArgs {
    const uint16_t* A;
    const uint16_t* B;
    float* C;                  // 16-byte aligned; C[b] at b * sC, row stride N
    int M, N, K;
    int64_t lda, ldb, sA, sB, sC;
    int row_blocks;            // ceil(M / 16)
    int per_batch;             // workgroups per batch (P)
};

constexpr int SK_WAVES = 8;
constexpr int SK_ROWS = 16;
constexpr int SK_LDS_MAX = 160 * 1024;
constexpr int SK_MAXB = 8;     // 16-column blocks per wave: N <= 16 * 8 * 8 = 1024 (6 when N <= 768)

typedef _Float16 skf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 skbf16x8 __attribute__((ext_vector_type(8)));

template <bool BF16>
__device__ __forceinline__ f32x4 sk_mfma(u32x4 a, u32x4 b, f32x4 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(skbf16x8, a), __builtin_bit_cast(skbf16x8, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(skf16x8, a), __builtin_bit_cast(skf16x8, b),
                                                      c, 0, 0, 0);
}

// Workgroup barrier ordering LDS only: its fences are limited to the local
// address space, so the waves' global stores stay in flight across it (a
// __syncthreads() would wait for every one of them to complete).
__device__ __forceinline__ void sk_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 16 bytes at p if the 8-element group starting at k lies inside K, else zeros
__device__ __forceinline__ u32x4 sk_load(const uint16_t* p, int k, int K) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (k < K) v = *reinterpret_cast<const u32x4*>(p);
    return v;
}

template <bool BF16, int KS, int MAXB>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_smallk_kernel(const SmallKArgs p) {
    extern __shared__ __attribute__((aligned(16))) float stage[];   // 16 N + 3 floats
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int b = blockIdx.x / p.per_batch, first = blockIdx.x % p.per_batch;
    const int N = p.N, K = p.K;
    const uint16_t* __restrict__ A = p.A + (int64_t)b * p.sA;
    const uint16_t* __restrict__ B = p.B + (int64_t)b * p.sB;
    const int kq = 8 * (lane >> 4);          // this lane's 8-element group within a k-step
    const int nb = (N + 15) / 16;            // 16-column blocks, dealt to the waves in turn
    const int mine = (nb - wave + SK_WAVES - 1) / SK_WAVES;

    // this wave's B fragments, for every row block of the workgroup
    u32x4 bf[MAXB][KS];
#pragma unroll
    for (int j = 0; j < MAXB; ++j) {
        const int col = min((wave + SK_WAVES * j) * 16 + (lane & 15), N - 1);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            bf[j][ks] = (u32x4){0u, 0u, 0u, 0u};
            if (j < mine) bf[j][ks] = sk_load(B + (int64_t)col * p.ldb + 32 * ks + kq, 32 * ks + kq, K);
        }
    }
    // the A rows of all this workgroup's row blocks into LDS, zero past K
    // (area: blocks x 16 rows x KS x 32 elements, after the staging area)
    const int nblk = (p.row_blocks - first + p.per_batch - 1) / p.per_batch;
    uint16_t* arows = reinterpret_cast<uint16_t*>(stage + ((SK_ROWS * N + 3 + 3) & ~3));
    constexpr int RE = KS * 32;   // elements per staged row
    for (int c = threadIdx.x; c < nblk * SK_ROWS * (RE / 8); c += 64 * SK_WAVES) {
        const int r = c / (RE / 8), k = (c % (RE / 8)) * 8;
        const int row = min((first + p.per_batch * (r / SK_ROWS)) * SK_ROWS + r % SK_ROWS, p.M - 1);
        *reinterpret_cast<u32x4*>(arows + r * RE + k) = sk_load(A + (int64_t)row * p.lda + k, k, K);
    }
    // every B fragment lands before the loop and is redefined by a pin: inside
    // the loop no instruction waits on a load the compiler tracks (such a wait
    // would be a vmcnt(0), which also waits for the stores in flight)
#pragma unroll
    for (int j = 0; j < MAXB; ++j)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm_pin(bf[j][ks]);
    __syncthreads();

    for (int i = 0; i < nblk; ++i) {
        const int rb = first + p.per_batch * i;
        const int i0 = rb * SK_ROWS, rows = min(SK_ROWS, p.M - i0);
        const int64_t g0 = (int64_t)b * p.sC + (int64_t)i0 * N;   // first float of this block's range
        const int s = (int)(g0 & 3);                              // LDS index of element t is t + s
        u32x4 a[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            a[ks] = *reinterpret_cast<const u32x4*>(arows + (i * SK_ROWS + (lane & 15)) * RE + 32 * ks + kq);
#pragma unroll
        for (int j = 0; j < MAXB; ++j) {
            if (j < mine) {
                f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) acc = sk_mfma<BF16>(a[ks], bf[j][ks], acc);
                const int col = (wave + SK_WAVES * j) * 16 + (lane & 15);
                if (col < N) {
#pragma unroll
                    for (int i2 = 0; i2 < 4; ++i2) {
                        const int r = 4 * (lane >> 4) + i2;
                        if (r < rows) stage[s + r * N + col] = acc[i2];
                    }
                }
            }
        }
        sk_lds_barrier();
        // the range [g0, g0 + L): e head floats up to the first 16-byte boundary,
        // whole aligned chunks, then the tail
        const int L = rows * N;
        const int e = min((4 - s) & 3, L);
        float* __restrict__ C = p.C + g0;
        const int t = threadIdx.x;
        if (t < e) C[t] = stage[s + t];
        const int chunks = (L - e) >> 2;
        for (int q = t; q < chunks; q += 64 * SK_WAVES)
            *reinterpret_cast<f32x4*>(C + e + 4 * q) = *reinterpret_cast<const f32x4*>(stage + s + e + 4 * q);
        const int tail0 = e + 4 * chunks;
        if (t < L - tail0) C[tail0 + t] = stage[s + tail0 + t];
        sk_lds_barrier();   // the staging area is read before the next block overwrites it; the stores drain
    }
}

bool smallk_supported(int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA, int64_t sB,
                      const void* A, const void* B, const void* C) {
    (void)M;
    return K <= 128 && K % 8 == 0 && ldc == N && N <= 16 * SK_WAVES * SK_MAXB && lda % 8 == 0 && ldb % 8 == 0 &&
           sA % 8 == 0 && sB % 8 == 0 && ((uintptr_t)A & 15) == 0 && ((uintptr_t)B & 15) == 0 &&
           ((uintptr_t)C & 15) == 0;
}

hipError_t launch_gemm_smallk(hipStream_t s, const void* A, int ab_dtype, const void* B, float* C, int batch, int M,
                              int N, int K, int64_t lda, int64_t ldb, int64_t sA, int64_t sB, int64_t sC, int num_cus) {
    SmallKArgs p{};
    p.A = (const uint16_t*)A;
    p.B = (const uint16_t*)B;
    p.C = C;
    p.M = M;
    p.N = N;
    p.K = K;
    p.lda = lda;
    p.ldb = ldb;
    p.sA = sA;
    p.sB = sB;
    p.sC = sC;
    p.row_blocks = (M + SK_ROWS - 1) / SK_ROWS;
    // workgroups per batch: each walks several row blocks of its batch (B is
    // loaded once per workgroup); MVLM_SMALLK_GROUPS overrides (sweeps)
    const int cus = num_cus > 0 ? num_cus : 256;
    int per = std::max(1, (cus + batch - 1) / batch);
    if (const char* e = std::getenv("MVLM_SMALLK_GROUPS")) {
        const int v = std::atoi(e);
        if (v > 0) per = v;
    }
    p.per_batch = std::max(1, std::min(p.row_blocks, per));
    const int ks = (K + 31) / 32;
    // LDS: the staging area (16 N + 3 floats, rounded to 16 bytes) and the A
    // rows of the workgroup's row blocks (16 rows x 32 ks elements each)
    auto lds_bytes = [&](int per_batch) {
        const int nblk = (p.row_blocks + per_batch - 1) / per_batch;
        return (uint32_t)(((SK_ROWS * N + 6) & ~3) * 4 + nblk * SK_ROWS * ks * 32 * 2);
    };
    while (lds_bytes(p.per_batch) > SK_LDS_MAX && p.per_batch < p.row_blocks) ++p.per_batch;
    const uint32_t lds = lds_bytes(p.per_batch);
    const dim3 grid((unsigned)(batch * p.per_batch)), block(64 * SK_WAVES);
    const bool bf = ab_dtype == MVLM_BF16;
#define SK_LAUNCH3(BFV, KSV, MB)                                                                                  \
    do {                                                                                                          \
        if (const hipError_t e = allow_dynamic_lds<gemm_smallk_kernel<BFV, KSV, MB>>(SK_LDS_MAX); e != hipSuccess) \
            return e;                                                                                             \
        launch_kernel(gemm_smallk_kernel<BFV, KSV, MB>, grid, block, lds, s, p);                                  \
    } while (0)
#define SK_LAUNCH(BFV, KSV)                                      \
    do {                                                         \
        if (N <= 16 * SK_WAVES * 6) SK_LAUNCH3(BFV, KSV, 6);     \
        else SK_LAUNCH3(BFV, KSV, SK_MAXB);                      \
    } while (0)
    switch (ks) {
        case 1: if (bf) SK_LAUNCH(true, 1); else SK_LAUNCH(false, 1); break;
        case 2: if (bf) SK_LAUNCH(true, 2); else SK_LAUNCH(false, 2); break;
        case 3: if (bf) SK_LAUNCH(true, 3); else SK_LAUNCH(false, 3); break;
        default: if (bf) SK_LAUNCH(true, 4); else SK_LAUNCH(false, 4); break;
    }
#undef SK_LAUNCH
#undef SK_LAUNCH3
    return hipGetLastError();
}

}  // namespace mvlm
