// Dequantizing skinny GEMM over GGUF Q8_0 / Q4_0 weights on the matrix cores:
// Y[m][n] = sum_k X[m][k] * w(n, k), 1 <= M <= 16, X and Y fp32 row-major.
//
// The reference plans this kernel (README.md:57, PLAN.md:65) but never wrote
// it.  With M > 1 the fp32 vector ALU would spend 2*M flops per streamed
// weight (M = 16: 42 GFLOP per Phi-1.5 step, ~270 us at the fp32 peak), so
// the products go to v_mfma_f32_16x16x32_bf16 instead, with no loss of
// precision:
//  * codes are small integers (Q8_0: -127..127, Q4_0: c - 8 in -8..7), exact
//    in bf16;
//  * x is split into three bf16 parts x = x1 + x2 + x3 (each the top 16 bits
//    of the remaining fp32 residual; the residuals are exact), which carries
//    24 significant bits, fp32's own precision, over fp32's exponent range;
//  * bf16 x bf16 products are exact in fp32 and the MFMA accumulates in fp32;
//  * the block scale d (fp16, exact in fp32) is applied once per block of 32
//    weights: acc += d * (sum over the block), as in the M = 1 kernel;
//  * Q4_0 multiplies the raw nibbles c and subtracts 8 * (sum of x over the
//    block), that sum coming from one more product of the split x with a
//    ones operand, shared by the block's row groups.
// One MFMA covers 16 weight rows x one block of 32 weights x 16 rows of X
// (rows m >= M are zero).  Operand layout of v_mfma_f32_16x16x32_bf16: lane l
// supplies A[l%16][8*(l/16) .. +7] and B[8*(l/16) .. +7][l%16]; accumulator
// register i of lane l is D[4*(l/16) + i][l%16].  Here A = X (row m = l%16)
// and B = w^T (weight row n0 + l%16), so lane l reads 8 consecutive codes of
// its weight row: Q8_0 bytes 8q..8q+7 of the block (q = l/16), Q4_0 the low
// (q < 2) or high (q >= 2) nibbles of bytes 8*(q&1)..+7 (byte j holds weights
// j and j + 16).
//
// A block of NW waves owns R groups of 16 weight rows; wave w takes the w-th
// NW-th of the K blocks and walks it in steps of G blocks (4, or 2 with four
// row groups).  Codes do not go straight to registers: in the MFMA layout a
// wave instruction would touch 16 rows x 32 bytes (16 partly used lines), and
// such loads ran at a fraction of HBM speed whatever the arithmetic.  Instead
// each step's codes of the wave's rows (16R rows x 32G bytes for Q8_0, x 16G
// bytes for Q4_0) are copied
// into the wave's own LDS slot with direct 16-byte loads (1 KiB contiguous
// per instruction), double-buffered, and read back per lane (ds_read_b64).
// The 16-byte pieces of each LDS row are XOR-swizzled with row bits so the
// 16 lanes of a read hit distinct banks.  The block's scales (all K) are
// staged once per block.  X goes straight to registers, one step ahead:
// each block's X registers are refilled for the next step as soon as that
// block's products are issued.
// The NW partial tiles meet in LDS.  Splitting K over blocks instead (to give
// small-N problems more blocks) would need a cross-block combine; on MI355X a
// device-scope release fence per block costs ~90 ns, serialized (1024 blocks:
// ~96 us), so small N gets 16-wave blocks instead.
#include "common.h"
#include "device_math.h"

#include <algorithm>

namespace mvlm {


typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8v;

// top 16 bits of two floats -> one packed bf16 pair (truncation)
__device__ __forceinline__ uint32_t pack_hi16(float lo_elem, float hi_elem) {
    return __builtin_amdgcn_perm(__float_as_uint(hi_elem), __float_as_uint(lo_elem), 0x07060302u);
}

// x[0..7] -> three bf16x8 parts with x = p1 + p2 + p3 (+ |residual| < 2^-24 |x|)
__device__ __forceinline__ void split3(const float (&x)[8], u32x4& p1, u32x4& p2, u32x4& p3) {
    float r1[8], r2[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float a = __uint_as_float(__float_as_uint(x[j]) & 0xFFFF0000u);
        r1[j] = x[j] - a;                                   // exact
        const float b = __uint_as_float(__float_as_uint(r1[j]) & 0xFFFF0000u);
        r2[j] = r1[j] - b;                                  // exact
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p1[j] = pack_hi16(x[2 * j], x[2 * j + 1]);
        p2[j] = pack_hi16(r1[2 * j], r1[2 * j + 1]);
        p3[j] = pack_hi16(r2[2 * j], r2[2 * j + 1]);
    }
}

// 8 small integers (exact in bf16) from 8 code bytes / nibbles.  Q4_0 gives
// the raw nibbles c (0..15): masked into bytes, one byte-to-float conversion
// each; the -8 of (c - 8) is applied per block through the block sums of x.
template <bool Q4>
__device__ __forceinline__ u32x4 codes_to_bf16(u32x2 raw, int q) {
    float v[8];
    if constexpr (Q4) {
        const int shift = (q >> 1) * 4;
        uint32_t lo = (raw[0] >> shift) & 0x0F0F0F0Fu, hi = (raw[1] >> shift) & 0x0F0F0F0Fu;
        // opaque to the compiler, which would otherwise fold each byte's
        // shift and mask into a bit-field extract per code in front of the
        // conversion; this way v_cvt_f32_ubyte{0..3} read the bytes directly
        asm_pin(lo);
        asm_pin(hi);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = (float)((lo >> (8 * j)) & 0xFFu);
            v[4 + j] = (float)((hi >> (8 * j)) & 0xFFu);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (float)(int8_t)(raw[j >> 2] >> (8 * (j & 3)));
    }
    u32x4 out;
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = pack_hi16(v[2 * j], v[2 * j + 1]);
    return out;
}

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a), __builtin_bit_cast(bf16x8v, b), c,
                                                   0, 0, 0);
}

constexpr size_t SKINNY_LDS_MAX = 160 * 1024;

// G = K blocks per step.
template <bool Q4, int G>
struct SkinnyLayout {
    static constexpr int BB = Q4 ? 16 : 32;           // code bytes per block per row
    static constexpr int CB = G * BB;                 // code bytes per row per step (32 / 64 / 128)
    static constexpr int P = CB / 16;                 // 16-byte pieces per row per step
    static constexpr int RPI = 64 / P;                // rows per direct-load instruction
    static constexpr int RSH = CB == 128 ? 1 : CB == 64 ? 2 : 3;   // 1 << RSH rows per 256 bytes
    static_assert(CB == 32 || CB == 64 || CB == 128, "step rows of 32, 64 or 128 bytes");
    // physical piece of logical piece p in LDS row r: the 16 rows of a read
    // land on distinct banks
    __device__ static int piece(int p, int r) { return p ^ ((r >> RSH) & (P - 1)); }
};

// LDS bytes of a block: the scales of its rows (all K), then two code slots
// per wave; the partial tiles of the final combine reuse the slots.
template <bool Q4, int R, int NW, int G>
__host__ __device__ constexpr int skinny_slot_bytes() { return 16 * R * SkinnyLayout<Q4, G>::CB; }
template <bool Q4, int R, int NW, int G>
static size_t skinny_lds_bytes(int K) {
    const size_t scale_region = ((size_t)16 * R * (K / 32) * 2 + 255) / 256 * 256;
    return scale_region + (size_t)NW * 2 * skinny_slot_bytes<Q4, R, NW, G>();
}

// One problem of a (possibly grouped) launch: Y[M][N] = X[M][K] w^T.
struct SkinnyProblem {
    const float* X;
    const uint8_t* codes;
    const uint16_t* scales;
    float* Y;
    int64_t ld;
    int N, K;
    int block_begin;               // first block of this problem in the grid
    int ep_on;
    Epilogue ep;
};
constexpr int SKINNY_MAX_GROUP = 8;
struct SkinnyGroup {
    SkinnyProblem p[SKINNY_MAX_GROUP];
    int count, M;
};

// XS: odd rows read their X halves in swapped order (M > 8, below).
template <bool Q4, int R, int NW, int G, bool XS>
__global__ __launch_bounds__(64 * NW, 4) void gemm_skinny_kernel(const SkinnyGroup g) {
    using L = SkinnyLayout<Q4, G>;
    constexpr int ROWS = 16 * R;
    constexpr int SLOT = skinny_slot_bytes<Q4, R, NW, G>();
    constexpr int NDMA = ROWS / L::RPI;               // direct loads per step
    static_assert(NDMA <= 63, "direct loads of one step must fit vmcnt");
    static_assert(2 * SLOT >= R * 1024, "the partial tiles of the combine must fit the code slots");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    int pi = 0;                                       // blocks are dealt to the problems in order
#pragma unroll
    for (int i = 1; i < SKINNY_MAX_GROUP; ++i)
        if (i < g.count && (int)blockIdx.x >= g.p[i].block_begin) pi = i;
    const SkinnyProblem& P = g.p[pi];
    const float* __restrict__ X = P.X;
    const uint8_t* __restrict__ codes = P.codes;
    const uint16_t* __restrict__ scales = P.scales;
    float* __restrict__ Y = P.Y;
    const int M = g.M, N = P.N, K = P.K;
    const int64_t ld = P.ld;

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l16 = lane & 15, q = lane >> 4;
    const int n0 = ((int)blockIdx.x - P.block_begin) * ROWS;
    const int nb = K >> 5;
    const int per = (nb + NW - 1) / NW;
    const int b0 = wave * per, b1 = min(b0 + per, nb);
    const int steps = b1 > b0 ? (b1 - b0 + G - 1) / G : 0;
    const int64_t row_bytes = (int64_t)nb * L::BB;

    // scales of rows n0 .. n0+ROWS-1 (contiguous in the scale array) with
    // 4-byte direct loads (a direct load writes lane i's data at base + 4i
    // whatever its width, so 2-byte loads would not pack).  Reads are clamped
    // to the last whole dword of the array (the allocation pads it); rows
    // past N read stale scales and are never stored.
    const int scale_bytes = ROWS * nb * 2;
    const int scale_region = (scale_bytes + 255) / 256 * 256;
    uint8_t* slots = lds + scale_region + wave * 2 * SLOT;
    const int64_t s_first = (int64_t)n0 * nb * 2, s_last = (((int64_t)N * nb * 2 - 1) & ~(int64_t)3);
    const uint8_t* scale_bytes_ptr = reinterpret_cast<const uint8_t*>(scales);
    for (int piece = wave; piece * 256 < scale_bytes; piece += NW) {
        const int64_t off = min(s_first + piece * 256 + lane * 4, s_last);
        __builtin_amdgcn_global_load_lds(scale_bytes_ptr + off, (lds_void*)(lds + piece * 256), 4, 0, 0);
    }

    // one step's direct loads: this wave's code rows into slot (step & 1).
    // Codes and X are read through buffer descriptors (32-bit offsets; the
    // host keeps both below 2 GiB on this path).
    const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(codes), 0, (int)min((int64_t)N * ld, (int64_t)0x7FFFFFFF), 0x00020000);
    const i32x4 xrs = raw_rsrc(X, (uint32_t)((int64_t)M * K * 4));
    const uint32_t xrow = (uint32_t)(((int64_t)min(l16, M - 1) * K + 8 * q) * 4);
    const int dma_row = lane / L::P, dma_piece = lane % L::P;
    auto issue_codes = [&](int step, int slot_idx) {
        const int kb = b0 + step * G;
        uint8_t* slot = slots + slot_idx * SLOT;
#pragma unroll
        for (int t = 0; t < NDMA; ++t) {
            const int r = t * L::RPI + dma_row;
            const int64_t row = min(n0 + r, N - 1);
            const int64_t off = min((int64_t)kb * L::BB + 16 * L::piece(dma_piece, r), row_bytes - 16);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(crs, (lds_void*)(slot + t * 1024), 16, (int)(row * ld + off), 0, 0, 0);
        }
    };
    // X of block g of one step into registers.  A lane's 8 floats are two
    // 16-byte halves of its row's 128-byte line.  With XS, lanes of odd rows
    // load the second half first, so the 16 lanes of a quarter-wave (16 rows,
    // one q) read two different offsets of their lines instead of one (the
    // vector cache serves many lines at one offset one after another: the
    // Q4_0 M = 16 step 827 -> 766 us, Q8_0 M = 16 895 -> 783 us, Q8_0 M = 12
    // 797 -> 760 us).  The halves are swapped back where the block is split;
    // at M <= 8 (at most 8 distinct lines) those selects cost more than the
    // conflicts (Q4_0 M = 5 707 -> 725 us), so XS is off there.
    const bool xodd = XS && (min(l16, M - 1) & 1) != 0;   // parity of the row actually read
    const int xsw = xodd ? 4 : 0;
    auto load_x = [&](int step, int g, u32x4 (&xg)[2]) {
        const int bb = min(b0 + step * G + g, nb - 1);
        xg[0] = asm_buffer_load_b128(xrs, xrow + (uint32_t)(32 * bb + xsw) * 4);
        xg[1] = asm_buffer_load_b128(xrs, xrow + (uint32_t)(32 * bb + 4 - xsw) * 4);
    };

    // Lanes whose X row is past M (clamped to row M - 1 above) only feed
    // output rows m >= M, which are never stored.
    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    u32x4 xr[G][2];                                   // X of the current step
    if (steps > 0) {
        issue_codes(0, 0);
#pragma unroll
        for (int g = 0; g < G; ++g) load_x(0, g, xr[g]);
    }
    asm_wait_vmcnt<0>();
    __syncthreads();                                  // the staged scales of every wave

    // LDS reads go through inline asm (the compiler would otherwise wait for
    // every in-flight direct load, including the next step's, before them)
    const uint32_t lds_base = lds_offset(lds);
    // Block g's X registers are refilled with the next step's X as soon as
    // its products are issued, so those loads overlap this step's work.  The
    // body is straight-line code (blocks past the wave's range get a zero
    // scale, the refill is unconditional and clamped in bounds): with no
    // branches the loop-carried X registers need no copies, which would read
    // them while their loads are still in flight.
    auto compute = [&](int step, u32x4 (&xr)[G][2], auto refill) {
        const int kb = b0 + step * G;
        const uint32_t slot = lds_offset(slots + (step & 1) * SLOT);
        u32x2 raw[G][R];
        uint32_t dh[G][R];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int lpiece = Q4 ? g : 2 * g + (q >> 1);
            const int bb = min(kb + g, b1 - 1);
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                const int r = 16 * rr + l16;
                raw[g][rr] = asm_lds_read_b64(slot + r * L::CB + 16 * L::piece(lpiece, r) + 8 * (q & 1));
                dh[g][rr] = asm_lds_read_u16(lds_base + 2 * (r * nb + bb));
            }
        }
        asm_wait_lgkmcnt<0>();
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                asm_pin(raw[g][rr]);
                asm_pin(dh[g][rr]);
            }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const bool live = kb + g < b1;            // uniform over the wave
            float x[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                x[j] = __uint_as_float(xodd ? xr[g][1][j] : xr[g][0][j]);
                x[4 + j] = __uint_as_float(xodd ? xr[g][0][j] : xr[g][1][j]);
            }
            u32x4 p1, p2, p3;
            split3(x, p1, p2, p3);
            f32x4 sx = {0.0f, 0.0f, 0.0f, 0.0f};      // Q4_0: sum of the block's x per X row
            if constexpr (Q4) {
                const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};   // bf16 1.0 pairs
                sx = mfma16(p1, ones, sx);
                sx = mfma16(p2, ones, sx);
                sx = mfma16(p3, ones, sx);
            }
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                const u32x4 w = codes_to_bf16<Q4>(raw[g][rr], q);
                f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
                c = mfma16(p1, w, c);
                c = mfma16(p2, w, c);
                c = mfma16(p3, w, c);
                if constexpr (Q4) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) c[i] = __builtin_fmaf(-8.0f, sx[i], c[i]);
                }
                const float d = live ? f16_bits_to_f32((uint16_t)dh[g][rr]) : 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[rr][i] = __builtin_fmaf(d, c[i], acc[rr][i]);
            }
            if constexpr (decltype(refill)::value) load_x(step + 1, g, xr[g]);
        }
    };

    // Per step: the next step's codes; waiting until only those remain in
    // flight covers this step's X (requested during the previous step, or
    // before the loop) and codes.  The last step is peeled: nothing is
    // requested for it, and it waits for everything.  X goes through
    // untracked loads, so the compiler adds no waits of its own.
    for (int step = 0; step + 1 < steps; ++step) {
        issue_codes(step + 1, (step + 1) & 1);
        asm_wait_vmcnt<NDMA>();
#pragma unroll
        for (int g = 0; g < G; ++g) {
            asm_pin(xr[g][0]);
            asm_pin(xr[g][1]);
        }
        compute(step, xr, std::true_type{});
    }
    asm_wait_vmcnt<0>();
    if (steps > 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            asm_pin(xr[g][0]);
            asm_pin(xr[g][1]);
        }
        compute(steps - 1, xr, std::false_type{});
    }

    // combine the NW partial tiles (reusing the code slots)
    __syncthreads();
    f32x4* part = reinterpret_cast<f32x4*>(lds + scale_region);
#pragma unroll
    for (int r = 0; r < R; ++r) part[(wave * R + r) * 64 + lane] = acc[r];
    __syncthreads();
    if (wave < R) {                                   // wave r sums row group r
        const int r = wave;
        f32x4 sum = part[r * 64 + lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            const f32x4 t = part[(w * R + r) * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) sum[i] += t[i];
        }
        const int n = n0 + 16 * r + l16;
        if (n < N) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * q + i;
                if (m < M) {
                    const int64_t idx = (int64_t)m * N + n;
                    Y[idx] = P.ep_on ? apply_epilogue(P.ep, sum[i], idx, n) : sum[i];
                }
            }
        }
    }
}

// Tile shape of a launch by its total 16-row groups.  Every wave reads its X
// slice from L2 for each K block (2 KiB per block at M = 16, 4x the Q4_0 code
// bytes of two row groups), so more row groups per wave means less X traffic
// per weight.  Q4_0 takes four row groups per wave (16-wave blocks, two K
// blocks per step, one block per CU) when those blocks fill the CUs in one
// round (Phi-1.5 QKV+fc1, 896 row groups: M = 16 14.5 -> 12.9 us, M = 8
// 12.7 -> 12.0 us); past one round the two-block-per-CU shape overlaps one
// block's prologue with the other's loop and wins (LM head, 3200 row groups:
// 41.0 us against 45.6 us).  Q8_0's codes are twice the bytes per weight, X
// weighs half as much, and the shorter per-block chain lost (M = 8 QKV+fc1
// 12.5 -> 13.5 us).  Then two row groups per block when that still gives
// every CU a block; fewer row groups than CUs get 16-wave blocks (more loads
// in flight per block), and so do Q4_0 launches of one to two row groups per
// CU (Phi-1.5 dense+fc2, 256 row groups: half the K steps per wave; Q4_0
// steps M = 5 708 -> 688 us, M = 8 728 -> 708 us, M = 16 768 -> 765 us, while
// Q8_0 lost: M = 16 781 -> 788 us).
enum SkinnyShape { SK_R4_W16, SK_R2_W8, SK_R1_W8, SK_R1_W16 };
static SkinnyShape skinny_shape(int64_t groups, int num_cus, bool q4) {
    if (q4 && groups >= 3 * (int64_t)num_cus && groups <= 4 * (int64_t)num_cus) return SK_R4_W16;
    if (groups >= 2 * (int64_t)num_cus) return SK_R2_W8;
    if (groups >= num_cus && !q4) return SK_R1_W8;
    return SK_R1_W16;
}

template <bool Q4>
static size_t skinny_lds_for(SkinnyShape sh, int K) {
    switch (sh) {
        case SK_R4_W16:
            if constexpr (Q4) return skinny_lds_bytes<Q4, 4, 16, 2>(K);
            return SKINNY_LDS_MAX + 1;                // Q4_0 only
        case SK_R2_W8: return skinny_lds_bytes<Q4, 2, 8, 4>(K);
        case SK_R1_W8: return skinny_lds_bytes<Q4, 1, 8, 4>(K);
        default: return skinny_lds_bytes<Q4, 1, 16, 4>(K);
    }
}

bool skinny_supported(int count, const mvlm_weight* const* ws, int num_cus) {
    if (num_cus <= 0) num_cus = 256;
    int64_t groups = 0;
    for (int i = 0; i < count; ++i) groups += (ws[i]->N + 15) / 16;
    const SkinnyShape sh = skinny_shape(groups, num_cus, count > 0 && ws[0]->dtype == MVLM_Q4_0);
    for (int i = 0; i < count; ++i) {
        const mvlm_weight* w = ws[i];
        if (!is_quant(w->dtype) || w->K % 32 != 0) return false;
        if (w->bytes > 0x7FFFFFFF || (int64_t)16 * w->K * 4 > 0x7FFFFFFF) return false;   // 32-bit buffer offsets
        const size_t lds = w->dtype == MVLM_Q4_0 ? skinny_lds_for<true>(sh, w->K) : skinny_lds_for<false>(sh, w->K);
        if (lds > SKINNY_LDS_MAX) return false;
    }
    return true;
}

template <bool Q4, int R, int NW, int G>
static hipError_t launch_skinny(hipStream_t s, SkinnyGroup& g) {
    const bool xs = g.M > 8;
    auto kernel = xs ? gemm_skinny_kernel<Q4, R, NW, G, true> : gemm_skinny_kernel<Q4, R, NW, G, false>;
    size_t lds = 0;
    unsigned blocks = 0;
    for (int i = 0; i < g.count; ++i) {
        lds = std::max(lds, skinny_lds_bytes<Q4, R, NW, G>(g.p[i].K));
        g.p[i].block_begin = (int)blocks;
        blocks += (unsigned)((g.p[i].N + 16 * R - 1) / (16 * R));
    }
    if (const hipError_t e = xs ? allow_dynamic_lds<gemm_skinny_kernel<Q4, R, NW, G, true>>((int)SKINNY_LDS_MAX)
                                : allow_dynamic_lds<gemm_skinny_kernel<Q4, R, NW, G, false>>((int)SKINNY_LDS_MAX);
        e != hipSuccess)
        return e;
    if (lds > SKINNY_LDS_MAX) return hipErrorInvalidValue;
    launch_kernel(kernel, dim3(blocks), dim3(64 * NW), (uint32_t)lds, s, g);
    return hipGetLastError();
}

// A grouped launch picks the shape from the row groups of all its problems.
template <bool Q4>
static hipError_t launch_skinny_shape(hipStream_t s, SkinnyGroup& g, int num_cus) {
    int64_t groups = 0;
    for (int i = 0; i < g.count; ++i) groups += (g.p[i].N + 15) / 16;
    switch (skinny_shape(groups, num_cus, Q4)) {
        case SK_R4_W16:
            if constexpr (Q4) return launch_skinny<Q4, 4, 16, 2>(s, g);
            return hipErrorInvalidValue;              // Q4_0 only
        case SK_R2_W8: return launch_skinny<Q4, 2, 8, 4>(s, g);
        case SK_R1_W8: return launch_skinny<Q4, 1, 8, 4>(s, g);
        default: return launch_skinny<Q4, 1, 16, 4>(s, g);
    }
}

static SkinnyProblem skinny_problem(const float* X, const mvlm_weight* W, float* Y) {
    SkinnyProblem p{};
    p.X = X;
    p.codes = (const uint8_t*)W->data;
    p.scales = (const uint16_t*)W->scales;
    p.Y = Y;
    p.ld = (int64_t)W->ld;
    p.N = W->N;
    p.K = W->K;
    return p;
}

hipError_t launch_gemm_skinny(hipStream_t s, const float* X, const mvlm_weight* W, float* Y, int M, int N, int K,
                              int num_cus, const Epilogue* ep) {
    if (M < 1 || M > 16 || K % 32 != 0 || !is_quant(W->dtype) || W->N != N || W->K != K) return hipErrorInvalidValue;
    if (num_cus <= 0) num_cus = 256;
    SkinnyGroup g{};
    g.count = 1;
    g.M = M;
    g.p[0] = skinny_problem(X, W, Y);
    if (ep && ep->any()) {
        g.p[0].ep = *ep;
        g.p[0].ep_on = 1;
    }
    if (W->dtype == MVLM_Q4_0) return launch_skinny_shape<true>(s, g, num_cus);
    return launch_skinny_shape<false>(s, g, num_cus);
}

hipError_t launch_gemm_skinny_group(hipStream_t s, int M, int count, const float* const* Xs,
                                    const mvlm_weight* const* ws, float* const* Ys, int num_cus,
                                    const Epilogue* eps) {
    if (M < 1 || M > 16 || count < 1 || count > SKINNY_MAX_GROUP) return hipErrorInvalidValue;
    if (num_cus <= 0) num_cus = 256;
    SkinnyGroup g{};
    g.count = count;
    g.M = M;
    for (int i = 0; i < count; ++i) {
        const mvlm_weight* W = ws[i];
        if (W->K % 32 != 0 || !is_quant(W->dtype) || W->dtype != ws[0]->dtype) return hipErrorInvalidValue;
        g.p[i] = skinny_problem(Xs[i], W, Ys[i]);
        if (eps && eps[i].any()) {
            g.p[i].ep = eps[i];
            g.p[i].ep_on = 1;
        }
    }
    if (ws[0]->dtype == MVLM_Q4_0) return launch_skinny_shape<true>(s, g, num_cus);
    return launch_skinny_shape<false>(s, g, num_cus);
}

}  // namespace mvlm
