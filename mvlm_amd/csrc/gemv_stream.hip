// Decode GEMV for every packed weight format, one or several independent
// problems per launch:  y_p[m][n] = sum_k x_p[m][k] * w_p(n, k), M = 1 (and,
// for quantized weights, M <= 4: batched decode, every weight chunk converted
// once and multiplied with the M rows of x).
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
#include "gemv_common.h"

#include <type_traits>

namespace mvlm {

// ---- the kernel ------------------------------------------------------------

// One problem of a grouped launch.  Chunk c of a row covers bytes
// [1024c, 1024c + 1024) of the row, lane l the 16 bytes at 1024c + 16l, i.e.
// weights [WPL*(64c + l), WPL*(64c + l + 1)).  K % WPL == 0, so a lane's vector
// lies entirely below K or entirely above it; lanes above K load the row's
// first vector instead (always in bounds) and discard the result, which keeps
// every load unconditional and lets them all issue before the first wait.
struct StreamProblem {
    const void* x;                 // [M][K]
    const uint8_t* codes;
    const uint16_t* scales;
    void* y;                       // [M][N]
    int64_t ld_bytes;
    int N, K, y_dtype;
    int M;                         // rows of x (1 for MX = 1; 2 for MX = 2; 3..4 for MX = 4)
    int shape;                     // index into kShapes
    int rows_per_block;            // block j owns rows [j*rows_per_block, (j+1)*rows_per_block) below N
    int block_begin;               // first block of this problem in the grid
    int ep_on;
    Epilogue ep;                   // applied to y when ep_on
};

constexpr int MAX_GROUP = 8;
#ifndef MVLM_STREAM_WAVES
#define MVLM_STREAM_WAVES 8
#endif
constexpr int NWAVE = MVLM_STREAM_WAVES;   // waves per block

struct StreamGroup {
    StreamProblem p[MAX_GROUP];
    int count;
};

// Work shape of one wave by row length in 1 KiB chunks: R rows x CW chunks,
// the row split over SPLIT waves when it is longer than CW chunks.  A wave
// keeps 4 to 8 loads of 16 bytes per lane in flight; whole rows per wave
// (SPLIT = 1) need no combine step.  The first kByLength shapes are chosen by
// row length; the last is shape 3 with two rows per wave, used with 2..4 rows
// of x (each wave then stages half as many x bytes per code byte; with one
// row of x it measured slower).
struct Shape { int max_chunks, R, CW, SPLIT; };
constexpr Shape kShapes[] = {{1, 4, 1, 1}, {2, 2, 2, 1}, {4, 1, 4, 1}, {8, 1, 4, 2}, {16, 1, 8, 2}, {8, 2, 4, 2},
                             {2, 1, 2, 1}};
constexpr int kNumShapes = 7, kByLength = 5, kBatchLong = 5, kFewRows2 = 6;
static_assert(sizeof(kShapes) / sizeof(kShapes[0]) == kNumShapes, "one kernel case per shape");

// The rows [row0, row0 + R) of one wave (those below the block's end rb1),
// its chunks wsub*CW ... of each, against MX rows of x (vector m staged at
// LDS byte m * x_stride; rows of x at or past M repeat row M-1 and are not
// stored).  x and the scales are already being staged into LDS (staging loads
// were issued before these and complete first).
template <class F, typename XT, int MX, int R, int CW, int SPLIT>
__device__ __forceinline__ void stream_rows(const StreamProblem& P, int rb0, int rb1, int64_t s_base, int x_stride,
                                            int x_region, const uint8_t* lds, float (*part)[4 * MX], int wave,
                                            int lane) {
    constexpr int WPL = F::WPL;
    constexpr int XB = WPL * (int)sizeof(XT);        // x bytes per lane per chunk
    constexpr int SL = XB >= 16 ? XB / 16 : 1;       // 16-byte LDS slots per lane per chunk
    const int K = P.K, nb = K >> 5;
    const int wsub = wave % SPLIT;
    const int row0 = rb0 + (wave / SPLIT) * R;
    const bool active = row0 < rb1;

    // the codes: every load of this wave before any arithmetic
    const uint8_t* rowp[R];
    int srow[R];                                      // row's scale byte offset in the staged region
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = (int64_t)min(row0 + r, rb1 - 1);
        rowp[r] = P.codes + row * P.ld_bytes;
        srow[r] = (int)(row * (nb * 2) - s_base);
    }
    u32x4 q[R][CW];
    int kk[CW];
    bool valid[CW];
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        const int c = wsub * CW + i;
        const int k = (64 * c + lane) * WPL;
        valid[i] = active && k < K;
        kk[i] = k < K ? k : 0;
#pragma unroll
        for (int r = 0; r < R; ++r)
            q[r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rowp[r] + (int64_t)kk[i] * 16 / WPL));
    }
    __builtin_amdgcn_sched_barrier(0);

    // LDS byte offsets of this lane's x slots.  A valid lane's slice of chunk c
    // starts at slot (64c + lane) * SL, and x_slot moves its slot v to
    // v ^ xt with xt = ((lane * SL) >> 4) & (SL - 1) for every c; a lane past K
    // reads the first slots instead (any in-bounds bytes: its result is
    // discarded).  So one add per read: xbase[i] + xoff[v].
    int xbase[CW], xoff[SL];
#pragma unroll
    for (int i = 0; i < CW; ++i) xbase[i] = valid[i] ? (64 * (wsub * CW + i) + lane) * SL * 16 : 0;
    {
        const int xt = ((lane * SL) >> 4) & (SL - 1);
#pragma unroll
        for (int v = 0; v < SL; ++v) xoff[v] = (v ^ xt) << 4;
    }

    // staging done for every wave -> x and scales from LDS, chunk by chunk
    wait_vmcnt<R * CW>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // Q4_0: the block sums of each row of x (the -8 offset's term, sxl[m][b]),
    // once per workgroup into LDS after the scales, instead of once per chunk,
    // row and wave
    constexpr bool kSumX = std::is_same_v<F, Q4Fmt>;
    const float* sxl = reinterpret_cast<const float*>(lds + x_region + ((P.rows_per_block * nb * 2 + 30 + 1023) & ~1023));
    if constexpr (kSumX) {
        for (int t = threadIdx.x; t < MX * nb; t += 64 * NWAVE) {
            const int m = MX == 1 ? 0 : t / nb, b = MX == 1 ? t : t - m * nb;
            const u32x4* xm = reinterpret_cast<const u32x4*>(lds + m * x_stride);
            XRaw<XT, WPL> xr;
#pragma unroll
            for (int v = 0; v < SL; ++v) {
                const u32x4 u = xm[x_slot<SL>(SL * b + v)];
                xr.d[4 * v + 0] = u[0]; xr.d[4 * v + 1] = u[1];
                xr.d[4 * v + 2] = u[2]; xr.d[4 * v + 3] = u[3];
            }
            const_cast<float*>(sxl)[t] = x_block_sum(xr);
        }
        // LDS-only fences around the barrier: the code loads stay in flight
        // (a full __syncthreads() would wait for them)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    float acc[R][MX];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MX; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        if constexpr (MX == 1) {   // one row of x: the x slice is read once per chunk
            XRaw<XT, WPL> xr;
            const int xbyte = kk[i] * (int)sizeof(XT);
            if constexpr (XB >= 16) {
#pragma unroll
                for (int v = 0; v < SL; ++v) {
                    const u32x4 u = *reinterpret_cast<const u32x4*>(lds + xbase[i] + xoff[v]);
                    xr.d[4 * v + 0] = u[0]; xr.d[4 * v + 1] = u[1];
                    xr.d[4 * v + 2] = u[2]; xr.d[4 * v + 3] = u[3];
                }
            } else {   // XB == 8
                const u32x2 u = *reinterpret_cast<const u32x2*>(lds + xbyte);
                xr.d[0] = u[0]; xr.d[1] = u[1];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint16_t dh = 0;
                if constexpr (F::QUANT)
                    dh = *reinterpret_cast<const uint16_t*>(lds + x_region + srow[r] + (kk[i] >> 5) * 2);
                float v;
                if constexpr (kSumX) v = chunk_dot_q4(q[r][i], dh, xr, sxl[kk[i] >> 5], acc[r][0]);
                else v = chunk_dot(F{}, q[r][i], dh, xr, acc[r][0]);
                acc[r][0] = valid[i] ? v : acc[r][0];
            }
            continue;
        }
#pragma unroll
        for (int m = 0; m < MX; ++m) {
            XRaw<XT, WPL> xr;
            const uint8_t* xl = lds + m * x_stride;
            const int xbyte = kk[i] * (int)sizeof(XT);
            if constexpr (XB >= 16) {
#pragma unroll
                for (int v = 0; v < SL; ++v) {
                    const u32x4 u = *reinterpret_cast<const u32x4*>(xl + xbase[i] + xoff[v]);
                    xr.d[4 * v + 0] = u[0]; xr.d[4 * v + 1] = u[1];
                    xr.d[4 * v + 2] = u[2]; xr.d[4 * v + 3] = u[3];
                }
            } else {   // XB == 8
                const u32x2 u = *reinterpret_cast<const u32x2*>(xl + xbyte);
                xr.d[0] = u[0]; xr.d[1] = u[1];
            }
            float sx = 0.0f;
            if constexpr (kSumX) sx = sxl[m * nb + (kk[i] >> 5)];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint16_t dh = 0;
                if constexpr (F::QUANT)
                    dh = *reinterpret_cast<const uint16_t*>(lds + x_region + srow[r] + (kk[i] >> 5) * 2);
                float v;
                if constexpr (kSumX) v = chunk_dot_q4(q[r][i], dh, xr, sx, acc[r][m]);
                else v = chunk_dot(F{}, q[r][i], dh, xr, acc[r][m]);
                acc[r][m] = valid[i] ? v : acc[r][m];
            }
        }
    }
    // the R x MX sums over the wave: lane j < R * MX ends with sum j = r * MX + m
    constexpr int NV = R * MX;
    float flat[NV];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MX; ++m) flat[r * MX + m] = acc[r][m];
    const float tot = wave_sum_lanes<NV>(flat, lane);
    const int jr = (lane & (NV - 1)) / MX, jm = (lane & (NV - 1)) % MX;

    // y[m][row] (and the epilogue's mul / residual [m][row], bias [row]),
    // the NV outputs of a wave stored by NV lanes at once
    auto store_row = [&](int row, int m, float v) {
        if constexpr (MX == 1) {
            store_out(P.y, row, P.ep_on ? apply_epilogue(P.ep, v, row, row) : v, P.y_dtype);
        } else {
            const int64_t idx = (int64_t)m * P.N + row;
            store_out(P.y, idx, P.ep_on ? apply_epilogue(P.ep, v, idx, row) : v, P.y_dtype);
        }
    };
    if constexpr (SPLIT == 1) {
        if (lane < NV && active && row0 + jr < rb1 && (MX == 1 || jm < P.M)) store_row(row0 + jr, jm, tot);
    } else {
        if (lane < NV) part[wave][lane] = tot;
        __syncthreads();
        if (wsub == 0 && lane < NV && active) {
            float v = part[wave][lane];
#pragma unroll
            for (int s = 1; s < SPLIT; ++s) v += part[wave + s][lane];
            if (row0 + jr < rb1 && (MX == 1 || jm < P.M)) store_row(row0 + jr, jm, v);
        }
    }
}

// A block of NWAVE waves owns a contiguous range of at most R * NWAVE / SPLIT
// rows of one problem.
// Per block, x and the rows' block scales are staged in LDS once (direct
// global->LDS loads), so each x element crosses the L2->CU path once per
// block rather than once per wave; the weight codes go straight to
// registers.  Issue order: x and scale staging, then every code load, then
// the wait for the staging alone (vmcnt counts in issue order), the block
// barrier, the LDS reads, and the wait for the codes.
template <class F, typename XT, int MX>
__global__ __launch_bounds__(64 * NWAVE, MX == 1 ? F::MIN_WAVES : F::MIN_WAVES_BATCH) void gemv_stream_kernel(
    const StreamGroup g) {
    constexpr int XB = F::WPL * (int)sizeof(XT);
    constexpr int SL = XB >= 16 ? XB / 16 : 1;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float part[NWAVE][4 * MX];

    int pi = 0;
#pragma unroll
    for (int i = 1; i < MAX_GROUP; ++i)
        if (i < g.count && (int)blockIdx.x >= g.p[i].block_begin) pi = i;
    const StreamProblem& P = g.p[pi];
    // the wave index is uniform: keep it in a scalar register so the staging
    // loops and row offsets are scalar code
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int N = P.N, K = P.K, nb = K >> 5;
    const int rb0 = ((int)blockIdx.x - P.block_begin) * P.rows_per_block;
    const int rb1 = min(rb0 + P.rows_per_block, N);

    // stage the MX rows of x (and the block's scales) in LDS
    // (x_bytes is a multiple of XB, so of 16 when XB >= 16)
    const int x_bytes = K * (int)sizeof(XT);
    const int x_stride = (x_bytes + 1023) & ~1023;
    const int x_region = MX * x_stride;
#pragma unroll
    for (int m = 0; m < MX; ++m)
        stage_to_lds<(XB >= 16 ? 16 : 4), SL, NWAVE>(lds + m * x_stride,
                                                    (const uint8_t*)P.x + (m == 0 ? 0 : (int64_t)min(m, P.M - 1) * x_bytes),
                                                    x_bytes, wave, lane);
    int64_t s_base = 0;                               // global byte offset of the first staged scale byte
    if constexpr (F::QUANT) {
        const int64_t s_begin = (int64_t)rb0 * (nb * 2);
        const int64_t s_end = (int64_t)rb1 * (nb * 2);
        s_base = s_begin & ~(int64_t)15;
        const int s_bytes = (int)((s_end - s_base + 15) & ~(int64_t)15);
        stage_to_lds<16, 1, NWAVE>(lds + x_region, (const uint8_t*)P.scales + s_base, s_bytes, wave, lane);
    }
    __builtin_amdgcn_sched_barrier(0);

    switch (P.shape) {   // uniform over the block
#define MVLM_SHAPE_CASE(i)                                                                               \
    case i:                                                                                              \
        stream_rows<F, XT, MX, kShapes[i].R, kShapes[i].CW, kShapes[i].SPLIT>(P, rb0, rb1, s_base, x_stride, \
                                                                               x_region, lds, part, wave, lane); \
        break;
        MVLM_SHAPE_CASE(0) MVLM_SHAPE_CASE(1) MVLM_SHAPE_CASE(2) MVLM_SHAPE_CASE(3) MVLM_SHAPE_CASE(4)
#undef MVLM_SHAPE_CASE
    case kFewRows2:
        if constexpr (MX == 1)
            stream_rows<F, XT, MX, kShapes[kFewRows2].R, kShapes[kFewRows2].CW, kShapes[kFewRows2].SPLIT>(
                P, rb0, rb1, s_base, x_stride, x_region, lds, part, wave, lane);
        break;
    case kBatchLong:
        if constexpr (MX > 1)
            stream_rows<F, XT, MX, kShapes[kBatchLong].R, kShapes[kBatchLong].CW, kShapes[kBatchLong].SPLIT>(
                P, rb0, rb1, s_base, x_stride, x_region, lds, part, wave, lane);
        break;
    }
}

// ---- launch configuration ----------------------------------------------------

static int weight_wpl(int dtype) {
    return dtype == MVLM_Q8_0 ? 16 : dtype == MVLM_Q4_0 ? 32 : 16 / (int)dtype_size(dtype);
}

// index into kShapes for this weight's row length and mx rows of x, -1 if
// rows are too long.  2-chunk rows with one row of x take one row per wave
// when two per wave would leave fewer workgroups than the device has CUs
// (num_cus > 0; num_cus == 0 keeps the by-length shape, whose LDS footprint
// bounds the one-row-per-wave variant's).
static int stream_shape(const mvlm_weight* w, int mx, int num_cus) {
    const int64_t chunks = (weight_row_bytes(w) + 1023) / 1024;
    for (int i = 0; i < kByLength; ++i)
        if (chunks <= kShapes[i].max_chunks) {
            if (mx > 1 && i == 3) return kBatchLong;
            if (mx == 1 && i == 1 && ((int64_t)w->N + 2 * NWAVE - 1) / (2 * NWAVE) < num_cus) return kFewRows2;
            return i;
        }
    return -1;
}

static int rows_per_block(int shape) { return kShapes[shape].R * (NWAVE / kShapes[shape].SPLIT); }

// LDS bytes of one block: x, then the block's scales plus the alignment
// slack of their start, each rounded to the 1 KiB pieces the staging writes.
// Scale reads reach up to 15 bytes past the scale array, which the weight
// allocation pads.
static size_t stream_lds_bytes(const mvlm_weight* w, int x_dtype, int shape, int mx = 1) {
    const size_t x_bytes = (size_t)w->K * dtype_size(x_dtype);
    size_t bytes = (size_t)mx * ((x_bytes + 1023) & ~(size_t)1023);
    if (is_quant(w->dtype))
        bytes += ((size_t)rows_per_block(shape) * (size_t)(w->K / 32) * 2 + 30 + 1023) & ~(size_t)1023;
    if (w->dtype == MVLM_Q4_0) bytes += (size_t)mx * (w->K / 32) * 4;   // block sums of each row of x
    return bytes;
}

constexpr size_t STREAM_LDS_MAX = 152 * 1024;

// Rows of x a launch's kernel carries: M = 2 has its own kernel (two fmas per
// converted weight), M = 3 and 4 share the four-row kernel (rows at or past M
// repeat row M - 1 and are not stored).
static int batch_mx(int M) { return M <= 1 ? 1 : M == 2 ? 2 : 4; }

bool stream_supported(const mvlm_weight* w, int M) {
    const int shape = stream_shape(w, M, 0);
    if (M > 1 && (M > 4 || !is_quant(w->dtype))) return false;
    return shape >= 0 && w->K % weight_wpl(w->dtype) == 0 &&
           stream_lds_bytes(w, MVLM_F32, shape, batch_mx(M)) <= STREAM_LDS_MAX;
}

int stream_max_group() { return MAX_GROUP; }

// Blocks per launch: each problem gets the fewest blocks whose row slots hold
// its rows.  (Spreading a problem over more, part-filled blocks to even out
// the bytes per CU was measured slower on MI355X: every block stages all of
// x, so x traffic grows with the block count, and part-filled blocks idle
// waves.  Computing block bounds by division, even once per block, also cost
// ~0.2 us per launch.)
static unsigned partition(StreamGroup& g) {
    unsigned begin = 0;
    for (int i = 0; i < g.count; ++i) {
        StreamProblem& p = g.p[i];
        p.rows_per_block = rows_per_block(p.shape);
        p.block_begin = (int)begin;
        begin += (unsigned)((p.N + p.rows_per_block - 1) / p.rows_per_block);
    }
    return begin;
}

template <class F, typename XT, int MX = 1>
static hipError_t launch_group(hipStream_t s, StreamGroup& g, size_t lds) {
    auto kernel = gemv_stream_kernel<F, XT, MX>;
    if (const hipError_t e = allow_dynamic_lds<gemv_stream_kernel<F, XT, MX>>((int)STREAM_LDS_MAX); e != hipSuccess)
        return e;
    const unsigned blocks = partition(g);
    launch_kernel(kernel, dim3(blocks), dim3(64 * NWAVE), (uint32_t)lds, s, g);
    return hipGetLastError();
}

template <class F>
static hipError_t launch_group_x(hipStream_t s, int x_dtype, StreamGroup& g, size_t lds) {
    switch (x_dtype) {
        case MVLM_F32: return launch_group<F, float>(s, g, lds);
        case MVLM_F16: return launch_group<F, __half>(s, g, lds);
        case MVLM_BF16: return launch_group<F, __hip_bfloat16>(s, g, lds);
        default: return hipErrorInvalidValue;
    }
}

// All problems share the weight dtype and x dtype (checked by the caller).
// M > 1 (2..4 rows of fp32 x per problem, quantized weights) uses the
// batched-x kernel.
hipError_t launch_gemv_stream_group(hipStream_t s, int count, const void* const* xs, int x_dtype,
                                    const mvlm_weight* const* ws, void* const* ys, const int* y_dtypes, int num_cus,
                                    const Epilogue* eps, int M) {
    if (count < 1 || count > MAX_GROUP || M < 1 || M > 4) return hipErrorInvalidValue;
    StreamGroup g{};
    g.count = count;
    const int dtype = ws[0]->dtype;
    if (M > 1 && (!is_quant(dtype) || x_dtype != MVLM_F32)) return hipErrorInvalidValue;
    size_t lds = 0;
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
        p.M = M;
        p.shape = stream_shape(w, M, num_cus > 0 ? num_cus : 256);
        if (eps && eps[i].any()) {
            p.ep = eps[i];
            p.ep_on = 1;
        }
        if (p.shape < 0 || w->dtype != dtype || (M > 1 && y_dtypes[i] != MVLM_F32)) return hipErrorInvalidValue;
        const size_t b = stream_lds_bytes(w, x_dtype, p.shape, batch_mx(M));
        lds = b > lds ? b : lds;
    }
    if (lds > STREAM_LDS_MAX) return hipErrorInvalidValue;
    if (M == 2) return dtype == MVLM_Q8_0 ? launch_group<Q8Fmt, float, 2>(s, g, lds) : launch_group<Q4Fmt, float, 2>(s, g, lds);
    if (M > 2) return dtype == MVLM_Q8_0 ? launch_group<Q8Fmt, float, 4>(s, g, lds) : launch_group<Q4Fmt, float, 4>(s, g, lds);
    switch (dtype) {
        case MVLM_Q8_0: return launch_group<Q8Fmt, float>(s, g, lds);
        case MVLM_Q4_0: return launch_group<Q4Fmt, float>(s, g, lds);
        case MVLM_F32: return launch_group_x<DenseFmt<float>>(s, x_dtype, g, lds);
        case MVLM_F16: return launch_group_x<DenseFmt<__half>>(s, x_dtype, g, lds);
        case MVLM_BF16: return launch_group_x<DenseFmt<__hip_bfloat16>>(s, x_dtype, g, lds);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_stream(hipStream_t s, const void* x, int x_dtype, const mvlm_weight* W, void* y,
                              int y_dtype, int num_cus, const Epilogue* ep) {
    return launch_gemv_stream_group(s, 1, &x, x_dtype, &W, &y, &y_dtype, num_cus, ep);
}

// Quantized weight, fp32 x [M][K] and y [M][N], 2 <= M <= 4.
hipError_t launch_gemv_stream_batch(hipStream_t s, const float* x, const mvlm_weight* W, float* y, int M,
                                    int num_cus, const Epilogue* ep) {
    if (M < 2 || M > 4 || !stream_supported(W, M)) return hipErrorInvalidValue;
    StreamGroup g{};
    g.count = 1;
    StreamProblem& p = g.p[0];
    p.x = x;
    p.codes = (const uint8_t*)W->data;
    p.scales = (const uint16_t*)W->scales;
    p.y = y;
    p.ld_bytes = weight_row_bytes(W);
    p.N = W->N;
    p.K = W->K;
    p.y_dtype = MVLM_F32;
    p.M = M;
    p.shape = stream_shape(W, M, num_cus > 0 ? num_cus : 256);
    if (ep && ep->any()) {
        p.ep = *ep;
        p.ep_on = 1;
    }
    const size_t lds = stream_lds_bytes(W, MVLM_F32, p.shape, batch_mx(M));
    if (M == 2) {
        if (W->dtype == MVLM_Q8_0) return launch_group<Q8Fmt, float, 2>(s, g, lds);
        if (W->dtype == MVLM_Q4_0) return launch_group<Q4Fmt, float, 2>(s, g, lds);
    } else {
        if (W->dtype == MVLM_Q8_0) return launch_group<Q8Fmt, float, 4>(s, g, lds);
        if (W->dtype == MVLM_Q4_0) return launch_group<Q4Fmt, float, 4>(s, g, lds);
    }
    return hipErrorInvalidValue;
}

}  // namespace mvlm
