// Decode GEMV (M = 1) for every packed weight format, one or several
// independent problems per launch:  y_p[n] = sum_k x_p[k] * w_p(n, k).
//
// Replaces gemv (src/kernels/gemm.cl:215-270) and adds the dequantizing
// Q8_0 / Q4_0 GEMV the reference plans (README.md:57).  A decode GEMV is one
// pass over the weight, so the kernel is organised around having all of a
// wave's HBM requests in flight before any arithmetic, and around few, large
// launches (a dependent launch costs ~1.6 us on MI355X, the time to stream
// ~10 MB):
//
//  * a "chunk" is one 16-byte vector per lane, 1 KiB per wave, of one weight
//    row: 4 fp32, 8 fp16/bf16, 16 Q8_0 codes (half a block) or 32 Q4_0 codes
//    (one block) per lane;
//  * a wave owns R rows x CW consecutive chunks (R*CW = 4: one contiguous
//    4 KiB region when a row is CW chunks long) and issues every code load,
//    every scale load and the matching x loads back to back; only then does
//    it convert and accumulate;
//  * rows longer than CW chunks are split over SPLIT = 2 or 4 waves of a
//    block (wave w takes chunks [w*CW, (w+1)*CW)); partial sums meet in LDS;
//  * one launch serves up to MAX_GROUP independent problems of the same
//    weight format (e.g. Phi-1.5's QKV and fc1, which read the same input, or
//    its dense and fc2 projections); blocks are dealt to problems in order.
// Codes become fp32 in registers: v_cvt_f32_i32 with a byte select for
// Q8_0, masked nibbles through v_cvt_f32_ubyte* for Q4_0.  The block scale is
// applied once per half block (Q8_0) or block (Q4_0):
//   Q8_0: acc += d * sum_j x_j q_j
//   Q4_0: acc += d * (sum_j x_j c_j - 8 sum_j x_j),  c_j the 4-bit code.
// This is the GGUF dequantization (w = d*q, w = (c-8)*d) with d factored out
// of each block: different rounding, same value within the fp32 tolerance.
#include "common.h"
#include "device_math.h"

namespace mvlm {

// ---- weight formats --------------------------------------------------------

template <typename WT>
struct DenseFmt {
    static constexpr int WPL = 16 / (int)sizeof(WT);   // weights per lane per chunk
    static constexpr bool QUANT = false;
};

struct Q8Fmt {
    static constexpr int WPL = 16;
    static constexpr bool QUANT = true;
};

struct Q4Fmt {
    static constexpr int WPL = 32;
    static constexpr bool QUANT = true;
};

// x values of one chunk as raw bits: E elements of XT in XD dwords.
template <typename XT, int E>
struct XRaw {
    static constexpr int XD = E * (int)sizeof(XT) / 4;
    uint32_t d[XD];
};

// Vector loads of E consecutive x elements at k (caller keeps k + E <= K).
template <typename XT, int E>
__device__ __forceinline__ void load_x_raw(const XT* __restrict__ x, int k, XRaw<XT, E>& out) {
    constexpr int XD = XRaw<XT, E>::XD;
    const uint32_t* p = reinterpret_cast<const uint32_t*>(x + k);
    if constexpr (XD % 4 == 0) {
#pragma unroll
        for (int v = 0; v < XD / 4; ++v) {
            u32x4 u = *reinterpret_cast<const u32x4*>(p + 4 * v);
            out.d[4 * v + 0] = u[0]; out.d[4 * v + 1] = u[1]; out.d[4 * v + 2] = u[2]; out.d[4 * v + 3] = u[3];
        }
    } else {   // XD == 2: four 16-bit elements
        u32x2 u = *reinterpret_cast<const u32x2*>(p);
        out.d[0] = u[0]; out.d[1] = u[1];
    }
}

template <typename XT, int E>
__device__ __forceinline__ float x_at(const XRaw<XT, E>& r, int j) {
    if constexpr (sizeof(XT) == 4) return __uint_as_float(r.d[j]);
    else return bits_to_f32<XT>((uint16_t)((j & 1) ? (r.d[j >> 1] >> 16) : (r.d[j >> 1] & 0xFFFFu)));
}

// dot of one chunk (16 bytes of weights) with its x values
template <typename WT, typename XT, int E>
__device__ __forceinline__ float chunk_dot(DenseFmt<WT>, u32x4 q, uint16_t, const XRaw<XT, E>& xr, float acc) {
    if constexpr (sizeof(WT) == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_fmaf(x_at(xr, j), __uint_as_float(q[j]), acc);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc = __builtin_fmaf(x_at(xr, 2 * j + 0), bits_to_f32<WT>((uint16_t)(q[j] & 0xFFFFu)), acc);
            acc = __builtin_fmaf(x_at(xr, 2 * j + 1), bits_to_f32<WT>((uint16_t)(q[j] >> 16)), acc);
        }
    }
    return acc;
}

template <typename XT, int E>
__device__ __forceinline__ float chunk_dot(Q8Fmt, u32x4 q, uint16_t dh, const XRaw<XT, E>& xr, float acc) {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) s = __builtin_fmaf(x_at(xr, j), (float)(int8_t)(q[j >> 2] >> (8 * (j & 3))), s);
    return __builtin_fmaf(f16_bits_to_f32(dh), s, acc);
}

// byte j of the block holds weight j (low nibble) and weight j + 16 (high nibble)
template <typename XT, int E>
__device__ __forceinline__ float chunk_dot(Q4Fmt, u32x4 q, uint16_t dh, const XRaw<XT, E>& xr, float acc) {
    float s = 0.0f, sx = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = nibbles_to_bytes(q[i]);
        const uint32_t hi = nibbles_to_bytes(q[i] >> 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s = __builtin_fmaf(x_at(xr, 4 * i + e), (float)((lo >> (8 * e)) & 0xFFu), s);
            s = __builtin_fmaf(x_at(xr, 16 + 4 * i + e), (float)((hi >> (8 * e)) & 0xFFu), s);
        }
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) sx += x_at(xr, j);
    return __builtin_fmaf(f16_bits_to_f32(dh), __builtin_fmaf(-8.0f, sx, s), acc);
}


// ---- the kernel ------------------------------------------------------------

// One problem of a grouped launch.  Chunk c of a row covers bytes
// [1024c, 1024c + 1024) of the row, lane l the 16 bytes at 1024c + 16l, i.e.
// weights [WPL*(64c + l), WPL*(64c + l + 1)).  K % WPL == 0, so a lane's vector
// lies entirely below K or entirely above it; lanes above K load the row's
// first vector instead (always in bounds) and discard the result, which keeps
// every load unconditional and lets them all issue before the first wait.
struct StreamProblem {
    const void* x;
    const uint8_t* codes;
    const uint16_t* scales;
    void* y;
    int64_t ld_bytes;
    int N, K, y_dtype, split;
    int block_begin;               // first block of this problem in the grid
};

constexpr int MAX_GROUP = 8;

struct StreamGroup {
    StreamProblem p[MAX_GROUP];
    int count;
};

template <class F, typename XT, int R, int CW>
__global__ __launch_bounds__(256) void gemv_stream_kernel(const StreamGroup g) {
    constexpr int WPL = F::WPL;
    int pi = 0;
#pragma unroll
    for (int i = 1; i < MAX_GROUP; ++i)
        if (i < g.count && (int)blockIdx.x >= g.p[i].block_begin) pi = i;
    const StreamProblem& P = g.p[pi];
    const XT* __restrict__ x = (const XT*)P.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int split = P.split, N = P.N, K = P.K;
    const int wsub = wave % split;
    const int row0 = (((int)blockIdx.x - P.block_begin) * (4 / split) + wave / split) * R;
    const int nb = K >> 5;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    if (row0 < N) {
        const uint8_t* rowp[R];
        const uint16_t* rows_s[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = (int64_t)min(row0 + r, N - 1);
            rowp[r] = P.codes + row * P.ld_bytes;
            rows_s[r] = P.scales + row * nb;
        }
        u32x4 q[R][CW];
        uint16_t dh[R][CW];
        XRaw<XT, WPL> xr[CW];
        bool valid[CW];
        // 1) every load of this wave is issued before any arithmetic
#pragma unroll
        for (int i = 0; i < CW; ++i) {
            const int c = wsub * CW + i;
            const int k = (64 * c + lane) * WPL;
            valid[i] = k < K;
            const int kk = valid[i] ? k : 0;   // byte offset in the row: kk * 16 / WPL
#pragma unroll
            for (int r = 0; r < R; ++r) {
                q[r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rowp[r] + (int64_t)kk * 16 / WPL));
                if constexpr (F::QUANT) dh[r][i] = rows_s[r][kk >> 5];
                else dh[r][i] = 0;
            }
            load_x_raw<XT, WPL>(x, kk, xr[i]);
        }
        // 2) convert and accumulate
#pragma unroll
        for (int i = 0; i < CW; ++i)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float v = chunk_dot(F{}, q[r][i], dh[r][i], xr[i], acc[r]);
                acc[r] = valid[i] ? v : acc[r];
            }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);

    if (split == 1) {                      // uniform over the block
        if (lane == 0 && row0 < N) {
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (row0 + r < N) store_out(P.y, row0 + r, acc[r], P.y_dtype);
        }
    } else {
        __shared__ float part[4][R];
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) part[wave][r] = acc[r];
        }
        __syncthreads();
        if (wsub == 0 && lane == 0 && row0 < N) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float v = part[wave][r];
                for (int s = 1; s < split; ++s) v += part[wave + s][r];
                if (row0 + r < N) store_out(P.y, row0 + r, v, P.y_dtype);
            }
        }
    }
}

// ---- launch configuration ----------------------------------------------------

// Rows per wave and chunks per wave for each format: R * CW = 4 loads of
// 16 bytes per lane.  A Q8_0 row of K = 2048 is 2 chunks (R = 2 rows per
// wave), a Q4_0 row of K = 2048 is 1 chunk (R = 4).  Rows per wave (Q8_0),
// measured on MI355X over the grouped Phi-1.5 decode step:
// R = 1: 599 us, 2: 428 us, 4: 439 us, 8: 470 us per step.
#ifndef MVLM_STREAM_R
#define MVLM_STREAM_R 2
#endif
template <class F> struct StreamShape { static constexpr int R = MVLM_STREAM_R, CW = 2; };
template <> struct StreamShape<Q4Fmt> { static constexpr int R = 2 * MVLM_STREAM_R, CW = 1; };

static int weight_wpl(int dtype) {
    return dtype == MVLM_Q8_0 ? 16 : dtype == MVLM_Q4_0 ? 32 : 16 / (int)dtype_size(dtype);
}
static int shape_cw(int dtype) { return dtype == MVLM_Q4_0 ? 1 : 2; }
static int shape_r(int dtype) { return dtype == MVLM_Q4_0 ? 2 * MVLM_STREAM_R : MVLM_STREAM_R; }

// waves sharing one row: ceil(chunks per row / CW), rounded up to 1, 2 or 4
static int stream_split(const mvlm_weight* w) {
    const int64_t chunks = (weight_row_bytes(w) + 1023) / 1024;
    const int cw = shape_cw(w->dtype);
    const int64_t s = (chunks + cw - 1) / cw;
    return s <= 1 ? 1 : s <= 2 ? 2 : s <= 4 ? 4 : 0;
}

bool stream_supported(const mvlm_weight* w) {
    return stream_split(w) > 0 && w->K % weight_wpl(w->dtype) == 0;
}

int stream_max_group() { return MAX_GROUP; }

template <class F, typename XT>
static hipError_t launch_group(hipStream_t s, const StreamGroup& g, unsigned blocks) {
    launch_kernel(gemv_stream_kernel<F, XT, StreamShape<F>::R, StreamShape<F>::CW>, dim3(blocks), dim3(256), 0, s, g);
    return hipGetLastError();
}

template <class F>
static hipError_t launch_group_x(hipStream_t s, int x_dtype, const StreamGroup& g, unsigned blocks) {
    switch (x_dtype) {
        case MVLM_F32: return launch_group<F, float>(s, g, blocks);
        case MVLM_F16: return launch_group<F, __half>(s, g, blocks);
        case MVLM_BF16: return launch_group<F, __hip_bfloat16>(s, g, blocks);
        default: return hipErrorInvalidValue;
    }
}

// All problems share the weight dtype and x dtype (checked by the caller).
hipError_t launch_gemv_stream_group(hipStream_t s, int count, const void* const* xs, int x_dtype,
                                    const mvlm_weight* const* ws, void* const* ys, const int* y_dtypes) {
    if (count < 1 || count > MAX_GROUP) return hipErrorInvalidValue;
    StreamGroup g{};
    g.count = count;
    const int dtype = ws[0]->dtype;
    const int R = shape_r(dtype);
    unsigned blocks = 0;
    for (int i = 0; i < count; ++i) {
        const mvlm_weight* w = ws[i];
        StreamProblem& p = g.p[i];
        p.x = xs[i];
        p.codes = (const uint8_t*)w->data;
        p.scales = (const uint16_t*)w->scales;
        p.y = ys[i];
        p.ld_bytes = weight_row_bytes(w);
        p.N = w->N;
        p.K = w->K;
        p.y_dtype = y_dtypes[i];
        p.split = stream_split(w);
        p.block_begin = (int)blocks;
        const int rows_per_block = R * (4 / p.split);
        blocks += (unsigned)((w->N + rows_per_block - 1) / rows_per_block);
    }
    switch (dtype) {
        case MVLM_Q8_0: return launch_group<Q8Fmt, float>(s, g, blocks);
        case MVLM_Q4_0: return launch_group<Q4Fmt, float>(s, g, blocks);
        case MVLM_F32: return launch_group_x<DenseFmt<float>>(s, x_dtype, g, blocks);
        case MVLM_F16: return launch_group_x<DenseFmt<__half>>(s, x_dtype, g, blocks);
        case MVLM_BF16: return launch_group_x<DenseFmt<__hip_bfloat16>>(s, x_dtype, g, blocks);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_stream(hipStream_t s, const void* x, int x_dtype, const mvlm_weight* W, void* y,
                              int y_dtype, int /*num_cus*/) {
    return launch_gemv_stream_group(s, 1, &x, x_dtype, &W, &y, &y_dtype);
}

}  // namespace mvlm
