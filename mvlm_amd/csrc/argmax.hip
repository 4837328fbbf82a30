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

#include <algorithm>
#include <climits>

namespace mvlm {

// The key as a signed integer that orders like the value it stands for: the
// magnitude bits with NaN payloads clamped to infinity's pattern and zero
// exponents to 0, negated for a set sign bit (sign-magnitude patterns of IEEE
// formats order like their values, so this needs no conversion to float).
template <int DT>
__device__ __forceinline__ int argmax_key_bits(uint32_t b) {
    constexpr int SIGN = DT == MVLM_F32 ? 31 : 15;
    constexpr uint32_t MAG = DT == MVLM_F32 ? 0x7FFFFFFFu : 0x7FFFu;
    constexpr uint32_t INF = DT == MVLM_F32 ? 0x7F800000u : DT == MVLM_F16 ? 0x7C00u : 0x7F80u;
    constexpr uint32_t MIN_NORMAL = DT == MVLM_F32 ? 0x00800000u : DT == MVLM_F16 ? 0x0400u : 0x0080u;
    uint32_t u = min(b & MAG, INF);                   // NaN -> inf
    u = u < MIN_NORMAL ? 0u : u;                      // zeros and subnormals -> 0
    const int neg = -(int)((b >> SIGN) & 1u);         // 0 or -1
    return ((int)u ^ neg) - neg;                      // -u when the sign bit is set
}

// below every key (keys lie in [-INF, INF]): a thread's first element always wins
constexpr int ARGMAX_NONE = INT_MIN;

__device__ __forceinline__ bool argmax_better(int k, int i, int bk, int bi) {
    return k > bk || (k == bk && i < bi);
}

constexpr int ARGMAX_THREADS = 1024;
constexpr int ARGMAX_BATCH = 8;       // 16-byte chunks in flight per thread

// element e of a 16-byte chunk
template <int DT>
__device__ __forceinline__ uint32_t chunk_elem(const u32x4& c, int e) {
    if constexpr (DT == MVLM_F32) return c[e];
    else return (c[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
}

// One workgroup per row.  VEC: the row starts 16-byte aligned and is read in
// 16-byte chunks (ARGMAX_BATCH per thread in flight); the last n % EPC
// elements, and every element when !VEC, are read one at a time.  Each thread
// visits its indices in increasing order, so its candidate is the first of
// its largest keys; the reductions break ties by the smaller index.
template <int DT, bool VEC>
__global__ __launch_bounds__(ARGMAX_THREADS) void argmax_kernel(const void* x, int n, int64_t ld, int* out) {
    __shared__ int wk[ARGMAX_THREADS / 64];
    __shared__ int wi[ARGMAX_THREADS / 64];
    constexpr int ES = DT == MVLM_F32 ? 4 : 2;
    constexpr int EPC = 16 / ES;
    const uint8_t* row = (const uint8_t*)x + (int64_t)blockIdx.x * ld * ES;
    int bk = ARGMAX_NONE;
    int bi = 0x7FFFFFFF;
    int scalar_from = 0;
    if constexpr (VEC) {
        const int nchunks = n / EPC;
        const u32x4* chunks = (const u32x4*)row;
        for (int base = threadIdx.x; base < nchunks; base += ARGMAX_THREADS * ARGMAX_BATCH) {
            u32x4 c[ARGMAX_BATCH];
#pragma unroll
            for (int u = 0; u < ARGMAX_BATCH; ++u) c[u] = chunks[min(base + u * ARGMAX_THREADS, nchunks - 1)];
#pragma unroll
            for (int u = 0; u < ARGMAX_BATCH; ++u) {
                const int ci = base + u * ARGMAX_THREADS;
                if (ci < nchunks) {
#pragma unroll
                    for (int e = 0; e < EPC; ++e) {
                        // a thread's indices only increase: a strictly larger key wins
                        const int k = argmax_key_bits<DT>(chunk_elem<DT>(c[u], e));
                        if (k > bk) {
                            bk = k;
                            bi = ci * EPC + e;
                        }
                    }
                }
            }
        }
        scalar_from = nchunks * EPC;
    }
    for (int i = scalar_from + threadIdx.x; i < n; i += ARGMAX_THREADS) {
        const uint32_t b = ES == 4 ? ((const uint32_t*)row)[i] : ((const uint16_t*)row)[i];
        const int k = argmax_key_bits<DT>(b);
        if (k > bk) {
            bk = k;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int ok = __shfl_xor(bk, off, 64);
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

// Split form for a few long rows (the token pick: one row of 51200 logits took
// 6.2-6.9 us on one workgroup, its key decode and compares on one CU's vector
// ALUs).  Row `row` is cut into gridDim.x slices of whole 16-byte chunks, one
// workgroup of ARGMAX_SPLIT_THREADS each (the last also takes the scalar
// tail); each workgroup folds its (key, index) candidate into the row's 64-bit
// word with a device-scope atomic max (the key, sign-flipped to order as an
// unsigned number, in the high half; 0x7FFFFFFF - index in the low half, so
// equal keys keep the smaller index) and, once that atomic has returned,
// counts itself in on the row's arrival counter.  The workgroup that arrives
// last reads the word, writes the index and sets word and counter back to
// zero for the next launch (both live in the device's sync words, zero
// between launches).
constexpr int ARGMAX_SPLIT_THREADS = 256;
constexpr int ARGMAX_SPLIT_ELEMS = 1600;    // elements per workgroup (about)
constexpr int ARGMAX_SPLIT_MAX = 64;        // workgroups per row

template <int DT, bool VEC>
__global__ __launch_bounds__(ARGMAX_SPLIT_THREADS) void argmax_split_kernel(const void* x, int n, int64_t ld,
                                                                             int* out, uint64_t* best,
                                                                             uint32_t* arrived) {
    __shared__ int wk[ARGMAX_SPLIT_THREADS / 64];
    __shared__ int wi[ARGMAX_SPLIT_THREADS / 64];
    constexpr int ES = DT == MVLM_F32 ? 4 : 2;
    constexpr int EPC = 16 / ES;
    const int row = (int)blockIdx.y, sl = (int)blockIdx.x, S = (int)gridDim.x;
    const uint8_t* base = (const uint8_t*)x + (int64_t)row * ld * ES;
    int bk = ARGMAX_NONE;
    int bi = 0x7FFFFFFF;
    // this slice: chunks [c0, c1) (VEC), else elements [e0, e1); the last
    // slice also takes the elements past the last whole chunk
    const int units = VEC ? n / EPC : n;
    const int u0 = (int)((int64_t)units * sl / S), u1 = (int)((int64_t)units * (sl + 1) / S);
    if constexpr (VEC) {
        const u32x4* chunks = (const u32x4*)base;
        for (int b0 = u0 + (int)threadIdx.x; b0 < u1; b0 += ARGMAX_SPLIT_THREADS * ARGMAX_BATCH) {
            u32x4 c[ARGMAX_BATCH];
#pragma unroll
            for (int u = 0; u < ARGMAX_BATCH; ++u) c[u] = chunks[min(b0 + u * ARGMAX_SPLIT_THREADS, u1 - 1)];
#pragma unroll
            for (int u = 0; u < ARGMAX_BATCH; ++u) {
                const int ci = b0 + u * ARGMAX_SPLIT_THREADS;
                if (ci < u1) {
#pragma unroll
                    for (int e = 0; e < EPC; ++e) {
                        const int k = argmax_key_bits<DT>(chunk_elem<DT>(c[u], e));
                        if (k > bk) {
                            bk = k;
                            bi = ci * EPC + e;
                        }
                    }
                }
            }
        }
    }
    const int e0 = VEC ? (sl == S - 1 ? units * EPC : n) : u0, e1 = VEC ? n : u1;
    for (int i = e0 + (int)threadIdx.x; i < e1; i += ARGMAX_SPLIT_THREADS) {
        const uint32_t b = ES == 4 ? ((const uint32_t*)base)[i] : ((const uint16_t*)base)[i];
        const int k = argmax_key_bits<DT>(b);
        if (k > bk) {
            bk = k;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const int ok = __shfl_xor(bk, off, 64);
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
        for (int w = 1; w < ARGMAX_SPLIT_THREADS / 64; ++w)
            if (argmax_better(wk[w], wi[w], bk, bi)) {
                bk = wk[w];
                bi = wi[w];
            }
        const uint64_t key = ((uint64_t)((uint32_t)bk ^ 0x80000000u) << 32) | (uint32_t)(0x7FFFFFFF - bi);
        const uint64_t prev = __hip_atomic_fetch_max(best + row, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" : : "v"(prev));      // the max has been performed before the count below
        const uint32_t old = __hip_atomic_fetch_add(arrived + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == (uint32_t)(S - 1)) {
            const uint64_t w = __hip_atomic_load(best + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            out[row] = 0x7FFFFFFF - (int)(uint32_t)w;
            __hip_atomic_store(best + row, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(arrived + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// slices per row of the split form, 1 for the one-workgroup form
int argmax_splits(int rows, int n) {
    if (rows > ARGMAX_SYNC_ROWS) return 1;
    return std::min(ARGMAX_SPLIT_MAX, n / ARGMAX_SPLIT_ELEMS);
}

template <int DT>
static void launch_dt(hipStream_t s, const void* x, int rows, int n, int64_t ld, int* out, void* sync) {
    constexpr int ES = DT == MVLM_F32 ? 4 : 2;
    const bool vec = ((uintptr_t)x & 15u) == 0 && (ld * ES) % 16 == 0;
    const int S = sync ? argmax_splits(rows, n) : 1;
    if (S > 1) {
        uint64_t* best = (uint64_t*)sync;
        uint32_t* arrived = (uint32_t*)(best + ARGMAX_SYNC_ROWS);
        const dim3 grid((unsigned)S, (unsigned)rows), block(ARGMAX_SPLIT_THREADS);
        if (vec) launch_kernel(argmax_split_kernel<DT, true>, grid, block, 0, s, x, n, ld, out, best, arrived);
        else launch_kernel(argmax_split_kernel<DT, false>, grid, block, 0, s, x, n, ld, out, best, arrived);
        return;
    }
    const dim3 grid((unsigned)rows), block(ARGMAX_THREADS);
    if (vec) launch_kernel(argmax_kernel<DT, true>, grid, block, 0, s, x, n, ld, out);
    else launch_kernel(argmax_kernel<DT, false>, grid, block, 0, s, x, n, ld, out);
}

hipError_t launch_argmax(hipStream_t s, const void* x, int dtype, int rows, int n, int64_t ld, int* out, void* sync) {
    switch (dtype) {
        case MVLM_F32: launch_dt<MVLM_F32>(s, x, rows, n, ld, out, sync); break;
        case MVLM_F16: launch_dt<MVLM_F16>(s, x, rows, n, ld, out, sync); break;
        case MVLM_BF16: launch_dt<MVLM_BF16>(s, x, rows, n, ld, out, sync); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mvlm
