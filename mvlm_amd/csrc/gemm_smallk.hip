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
// 16 waves split the columns (16-column blocks dealt in turn, at most 4 per
// wave) and load the B fragments of their columns into registers once, for
// every row block they compute: B (K of attention) is read from L2 once per
// workgroup instead of once per row block.  The A rows of all its row blocks
// are staged into LDS first, so the row-block loop issues no vector loads and
// never waits on the vector-memory counter: the stores of every block stay in
// flight while the next blocks are computed (loads and stores share that
// counter, so a wait for a load would also wait for them).
//
// Schedule.  Per-phase s_memrealtime stamps of an instrumented copy (SigLIP
// scores, 16 workgroups per batch) showed the earlier 8-wave form spending
// ~3.7 us before its first product, then ~1.2 us of products and ~0.8 us of
// store issue per row block, one after another.  Now: 16 waves share the
// columns (half the products per wave); the A loads are issued before B's and
// written to LDS while B's are in flight, and the first block's products wait
// for their own B fragments only (loads return in order); a block's
// accumulator chains are issued together before any is written to LDS; the
// staging area is double-buffered, so one barrier per block separates the
// products of block i + 1 from the stores of block i; the store phase issues
// all its LDS reads before its stores; and the stores write through the XCD's
// L2 (sc1), so the 34 MB of scores do not sit in L2 as dirty lines that the
// end of the kernel has to write back.  Measured on the SigLIP shape, 16
// copies in one graph: 13.2 us (8 waves) -> 11.8 (write-through stores) ->
// 10.6 us.  The row blocks then follow each other ~1.6 us apart, which is the
// time HBM takes to absorb one round of them (12 MB over the 256 workgroups):
// what is left above the write time is the ~4 us before the first stores.
//
// Products: v_mfma_f32_16x16x32_{f16,bf16} with B's fragment as the first
// operand, so the accumulator holds the block transposed.  Operand layout:
// lane l supplies B^T[l%16][8*(l/16) .. +7] and A[l%16][8*(l/16) .. +7] for
// k-step ks (K offset 32 ks); accumulator register i of lane l is
// C[l%16][4*(l/16) + i]: four consecutive columns of one row, written to LDS
// as two 8-byte pairs (the 16 rows of a block are N floats apart, 25 banks
// for N = 729, so a quarter-wave's pairs fall in distinct banks).
// K is a multiple of 8: an 8-element group is inside K or past it, and groups
// past K are zero in registers (their buffer loads are out of range).  Rows of A past M load row M - 1 and columns of B past N
// load column N - 1; their products are never stored.  fp16/bf16 products are
// exact in fp32; the matrix core's accumulation order differs from an fma
// chain in ascending k, within the 1e-3 relative bound of 16-bit inputs.
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

constexpr int SK_WAVES = 16;
constexpr int SK_ROWS = 16;
constexpr int SK_LDS_MAX = 160 * 1024;
constexpr int SK_MAXB = 4;     // 16-column blocks per wave: N <= 16 * 16 * 4 = 1024 (3 when N <= 768)
constexpr int SK_A_EARLY = 1;  // A groups per thread loaded before B's loads
constexpr int SK_CPOL_WT = 16; // sc1: the store writes through the XCD's L2

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

// The 8-element group starting at element k of the row at element offset
// `row` of an operand (raw buffer `r`): a group past K reads at an offset
// beyond the buffer's size, which returns zeros and moves no data.  No branch
// around the load, so the compiler counts the loads in flight exactly and
// waits for each one alone.  (Reading the row's last group inside K instead
// made the load phase ~0.7 us longer: the first loads' time is set by the
// bytes the CUs take in.)
constexpr int SK_OOB = 0x7FFFFFF0;   // beyond every operand (sizes are checked below 2^30 bytes)
__device__ __forceinline__ u32x4 sk_load(__amdgpu_buffer_rsrc_t r, int row, int k, int K) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, k < K ? 2 * (row + k) : SK_OOB, 0, 0));
}

template <bool BF16, int KS, int MAXB>
__global__ __launch_bounds__(64 * SK_WAVES) void gemm_smallk_kernel(const SmallKArgs p) {
    // LDS: two staging areas of SA floats (16 N + 3 each, rounded up to 16
    // bytes), the A rows of the workgroup's row blocks, a spare 16-byte slot
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // workgroup x runs on XCD x % 8: the workgroups of one batch are numbered
    // so that they share an XCD (and its L2 copy of B) when the grid allows
    int w = blockIdx.x;
    if ((gridDim.x & 7) == 0) w = (w & 7) * (gridDim.x >> 3) + (w >> 3);
    const int b = w / p.per_batch, first = w % p.per_batch;
    const int N = p.N, K = p.K, M = p.M;
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.A + (int64_t)b * p.sA), 0, (int)(2 * ((int64_t)(M - 1) * p.lda + K)), 0x00020000);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.B + (int64_t)b * p.sB), 0, (int)(2 * ((int64_t)(N - 1) * p.ldb + K)), 0x00020000);
    const int kq = 8 * (lane >> 4);          // this lane's 8-element group within a k-step
    const int nb = (N + 15) / 16;            // 16-column blocks, dealt to the waves in turn
    const int mine = (nb - wave + SK_WAVES - 1) / SK_WAVES;
    const int nblk = (p.row_blocks - first + p.per_batch - 1) / p.per_batch;
    if (nblk <= 0) return;
    const int SA = (SK_ROWS * N + 3 + 3) & ~3;
    uint16_t* arows = reinterpret_cast<uint16_t*>(smem + 2 * SA);
    constexpr int RE = KS * 32;              // elements per staged A row
    constexpr int GPR = RE / 8;              // 8-element groups per staged A row
    const int agroups = nblk * SK_ROWS * GPR;
    auto a_row = [&](int c) {                // element offset of the A row of staged group c
        const int r = c / GPR;
        return min((first + p.per_batch * (r / SK_ROWS)) * SK_ROWS + r % SK_ROWS, M - 1) * (int)p.lda;
    };

    // 1. the first A groups of this thread, then every B fragment of this wave
    //    (columns of blocks past `mine` load column N - 1 and are never stored)
    //    (a wave with no A group left loads nothing: its one load would wait
    //    behind the other waves' loads in the CU's queue, ~2.4 us in the
    //    stamped copy, and the barrier after the staging waits for every wave)
    u32x4 ae[SK_A_EARLY];
#pragma unroll
    for (int u = 0; u < SK_A_EARLY; ++u) {
        const int c = (int)threadIdx.x + 64 * SK_WAVES * u;
        if (64 * (wave + SK_WAVES * u) < agroups) ae[u] = sk_load(ar, a_row(min(c, agroups - 1)), (min(c, agroups - 1) % GPR) * 8, K);
    }
    u32x4 bf[MAXB][KS];
#pragma unroll
    for (int j = 0; j < MAXB; ++j) {
        const int col = min((wave + SK_WAVES * j) * 16 + (lane & 15), N - 1);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) bf[j][ks] = sk_load(br, col * (int)p.ldb, 32 * ks + kq, K);
    }
    // 2. A into LDS (zero past K); groups beyond the early ones (many row blocks
    //    per workgroup) are loaded here, after B's loads
    // (a group past the last goes to a spare slot after the A rows: the write
    // has no branch, so the compiler cannot sink its load below B's)
#pragma unroll
    for (int u = 0; u < SK_A_EARLY; ++u) {
        const int c = (int)threadIdx.x + 64 * SK_WAVES * u;
        const int slot = c < agroups ? (c / GPR) * RE + (c % GPR) * 8 : agroups * 8;
        if (64 * (wave + SK_WAVES * u) < agroups) *reinterpret_cast<u32x4*>(arows + slot) = ae[u];
    }
    for (int c = (int)threadIdx.x + 64 * SK_WAVES * SK_A_EARLY; c < agroups; c += 64 * SK_WAVES)
        *reinterpret_cast<u32x4*>(arows + (c / GPR) * RE + (c % GPR) * 8) = sk_load(ar, a_row(c), (c % GPR) * 8, K);
    sk_lds_barrier();

    // products of row block i into staging area buf (LDS index of the block's
    // element t is t + its shift)
    auto compute = [&](int i, float* stage) {
        const int i0 = (first + p.per_batch * i) * SK_ROWS, rows = min(SK_ROWS, M - i0);
        const int s = (int)(((int64_t)b * p.sC + (int64_t)i0 * N) & 3);
        u32x4 a[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            a[ks] = *reinterpret_cast<const u32x4*>(arows + (i * SK_ROWS + (lane & 15)) * RE + 32 * ks + kq);
        f32x4 acc[MAXB];
#pragma unroll
        for (int j = 0; j < MAXB; ++j) {
            acc[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) acc[j] = sk_mfma<BF16>(bf[j][ks], a[ks], acc[j]);
        }
        // lane l holds row l % 16, columns 4 (l / 16) .. + 3 of each of its blocks
        const int r = lane & 15;
        float* row = stage + s + r * N;
#pragma unroll
        for (int j = 0; j < MAXB; ++j) {
            const int col = (wave + SK_WAVES * j) * 16 + 4 * (lane >> 4);
            if (j < mine && r < rows) {
                if (col + 3 < N) {
#pragma unroll
                    for (int i2 = 0; i2 < 4; ++i2) row[col + i2] = acc[j][i2];
                } else {
#pragma unroll
                    for (int i2 = 0; i2 < 4; ++i2)
                        if (col + i2 < N) row[col + i2] = acc[j][i2];
                }
            }
        }
    };
    // the range [g0, g0 + L) of row block i: e head floats up to the first
    // 16-byte boundary, whole aligned chunks, then the tail
    auto store = [&](int i, const float* stage) {
        const int i0 = (first + p.per_batch * i) * SK_ROWS, rows = min(SK_ROWS, M - i0);
        const int64_t g0 = (int64_t)b * p.sC + (int64_t)i0 * N;
        const int s = (int)(g0 & 3);
        const int L = rows * N;
        const int e = min((4 - s) & 3, L);
        const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(p.C + g0, 0, L * 4, 0x00020000);
        const int t = threadIdx.x;
        const int chunks = (L - e) >> 2;
        // s + e is 0 or 4 whenever a chunk exists: the chunks' LDS reads are 16-byte aligned
        const float* src = stage + ((s + e + 3) & ~3);
        constexpr int U = MAXB;              // chunks per thread: 16 N / 4 / 1024 = N / 256 <= MAXB
        f32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = t + 64 * SK_WAVES * u;
            if (q < chunks) v[u] = *reinterpret_cast<const f32x4*>(src + 4 * q);
        }
        if (t < e) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(stage[s + t]), cr, 4 * t, 0, SK_CPOL_WT);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int q = t + 64 * SK_WAVES * u;
            if (q < chunks)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v[u]), cr, 4 * (e + 4 * q), 0,
                                                       SK_CPOL_WT);
        }
        const int tail0 = e + 4 * chunks;
        if (t < L - tail0)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(stage[s + tail0 + t]), cr, 4 * (tail0 + t), 0,
                                                  SK_CPOL_WT);
    };

    compute(0, smem);
    sk_lds_barrier();
    // every B fragment has landed (block 0 used them all) and is redefined by a
    // pin: inside the loop no instruction waits on a load the compiler tracks
    // (such a wait would be a vmcnt(0), which also waits for the stores in flight)
#pragma unroll
    for (int j = 0; j < MAXB; ++j)
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) asm_pin(bf[j][ks]);
    for (int i = 0; i < nblk; ++i) {
        store(i, smem + (i & 1) * SA);
        if (i + 1 < nblk) compute(i + 1, smem + ((i + 1) & 1) * SA);
        sk_lds_barrier();   // block i + 1 staged before its stores; block i's area read before block i + 2 reuses it
    }
}

bool smallk_supported(int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA, int64_t sB,
                      const void* A, const void* B, const void* C) {
    // operand rows addressed with 32-bit byte offsets, below the out-of-range offset
    const bool offsets = (int64_t)M * lda * 2 < (1 << 30) && (int64_t)N * ldb * 2 < (1 << 30);
    return offsets && K <= 128 && K % 8 == 0 && ldc == N && N <= 16 * SK_WAVES * SK_MAXB && lda % 8 == 0 && ldb % 8 == 0 &&
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
    // LDS: two staging areas (16 N + 3 floats each, rounded to 16 bytes), the A
    // rows of the workgroup's row blocks (16 rows x 32 ks elements each) and a
    // spare 16-byte slot
    auto lds_bytes = [&](int per_batch) {
        const int nblk = (p.row_blocks + per_batch - 1) / per_batch;
        return (uint32_t)(2 * ((SK_ROWS * N + 6) & ~3) * 4 + nblk * SK_ROWS * ks * 32 * 2 + 16);
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
        if (N <= 16 * SK_WAVES * 3) SK_LAUNCH3(BFV, KSV, 3);     \
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
