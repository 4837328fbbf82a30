// Prefill / vision GEMM on CDNA4 matrix cores:
//   C[b][m][n] = sum_k A[b][m][k] * B[b][n][k]     (NT: both operands K-contiguous)
// A and B fp16 or bf16, fp32 accumulation, C stored fp32 / fp16 / bf16.
//
// Replaces gemm_image (src/kernels/gemm.cl:157-200) as the prefill path
// (dispatch_gemm_image, src/engine/compute.cpp:90-120; every projection in
// src/models/moondream2.cpp:374-508) and serves the batched attention scores
// Q*K^T (the dot of src/kernels/attention.cl:84-88).
//
// Structure.  A block of WGM x WGN waves owns a BM x BN tile of C; each wave a
// (BM/WGM) x (BN/WGN) sub-tile of 32x32 v_mfma_f32_32x32x16 tiles.
// K advances in 64-wide stages held in an LDS ring of STAGES slots:
//  * global -> LDS with global_load_lds_dwordx4: one wave instruction moves
//    8 rows x 128 bytes (a 64-element K slice of 8 rows) straight into LDS,
//    no registers involved, so up to STAGES-1 stages are in flight while the
//    MFMAs work on the oldest;
//  * LDS rows are 128 bytes; the 16-byte slot s of row r is stored at slot
//    s ^ ((r >> 1) & 7).  gfx950's LDS serves a ds_read_b128 16 lanes at a
//    time from 64 four-byte banks (a 256-byte period, two rows), so the 16
//    rows read by one phase must occupy 16 distinct (row parity, slot) pairs;
//    an (r & 7) swizzle leaves rows r and r+8 on the same banks (measured:
//    half of all LDS cycles were bank conflicts).  The swizzle is applied on
//    the global side: lane i of a load instruction writes LDS bytes
//    [16i, 16i+16) of its 8-row group g and so fetches logical slot
//    (i & 7) ^ ((4g + (i >> 4)) & 7);
//  * one barrier per stage: after it, the slot computed in the previous
//    iteration is refilled.
// Rows beyond M / N are clamped to the last valid row (their products land in
// outputs that are never stored).  K beyond the operand's readable width is
// zero-filled by a guarded load path used only for the last stage.
// Operand layout of v_mfma_f32_32x32x16_{f16,bf16}: lane l supplies
// A[l%32][8*(l/32) .. +7] and B^T[l%32][8*(l/32) .. +7]; accumulator register
// r of lane l is C[8*(r/4) + 4*(l/32) + r%4][l%32].
#include "common.h"
#include "device_math.h"

#include <cstdio>
#include <cstdlib>

namespace mvlm {

constexpr int BK = 64;       // K per stage
constexpr int ROWH = BK;     // elements per LDS row (128 bytes)

struct GemmArgs {
    const uint16_t* A;
    const uint16_t* B;
    void* C;
    int c_dtype;
    int M, N, K;
    int64_t lda, ldb, ldc, sA, sB, sC;
    int kread_b;        // B rows are readable (zero padded) up to this K (>= K)
    int tiles_m, tiles_n;
    Epilogue ep;        // applied when ep_on (mul / res indexed like C)
    int ep_on;
};

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Direct loads of one operand's stage: ROWS rows starting at tile row r0,
// K columns [k0, k0+64).  Wave w of NW issues 8-row groups w, w+NW, ...
template <int ROWS, int NW>
__device__ __forceinline__ void stage_direct(const uint16_t* __restrict__ base, int64_t ld, int r0, int rmax, int k0,
                                             uint16_t* lds, int wave, int lane) {
    // logical 16-byte slot this lane fetches: its LDS row is 8g + (lane >> 3)
    // with g = wave + NW*t (NW even), so (row >> 1) & 7 = (4 * (wave & 1) + (lane >> 4)) & 7
    const int ls = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
    static_assert((ROWS / 8) % NW == 0, "8-row groups must split evenly over the waves");
#pragma unroll
    for (int t = 0; t < ROWS / (8 * NW); ++t) {
        const int g = wave + NW * t;
        const int r = min(r0 + 8 * g + (lane >> 3), rmax);
        const uint16_t* src = base + (int64_t)r * ld + k0 + ls * 8;
        asm_global_load_lds_b128(src, __builtin_amdgcn_readfirstlane(lds_offset(lds + 8 * g * ROWH)));
    }
}

// Guarded loads of the last stage: 16-byte chunks at or beyond kread are zero.
template <int ROWS, int NW>
__device__ __forceinline__ void stage_guarded(const uint16_t* __restrict__ base, int64_t ld, int r0, int rmax, int k0,
                                              int kread, uint16_t* lds, int wave, int lane) {
    const int ls = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
    static_assert((ROWS / 8) % NW == 0, "8-row groups must split evenly over the waves");
#pragma unroll
    for (int t = 0; t < ROWS / (8 * NW); ++t) {
        const int g = wave + NW * t;
        const int r = min(r0 + 8 * g + (lane >> 3), rmax);
        const int k = k0 + ls * 8;
        u32x4 v = {0, 0, 0, 0};
        if (k < kread) v = *reinterpret_cast<const u32x4*>(base + (int64_t)r * ld + k);
        *reinterpret_cast<u32x4*>(lds + 8 * g * ROWH + lane * 8) = v;
    }
}

template <bool BF16, int BM, int BN, int STAGES, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_mfma_kernel(const GemmArgs p) {
    constexpr int NW = WGM * WGN;                // waves per block (WGM x WGN grid)
    constexpr int WM = BM / WGM, WN = BN / WGN;  // wave sub-tile
    constexpr int TM = WM / 32, TN = WN / 32;    // 32x32 MFMA tiles per wave
    constexpr int LA = (BM / 8 + BN / 8) / NW;   // direct-load instructions per wave per stage
    constexpr int SLOT = (BM + BN) * ROWH;       // elements per ring slot
    static_assert(TM + TN <= 15, "fragment reads must fit the lgkmcnt field");
    __shared__ __attribute__((aligned(1024))) uint16_t smem[STAGES * SLOT];

    // Tile order: blocks are dealt round-robin to the 8 XCDs; give each XCD a
    // contiguous run of tiles in which the M tiles of one N tile are adjacent,
    // so the blocks reading the same weight tile share that XCD's L2.
    const int tiles = p.tiles_m * p.tiles_n;
    int t = blockIdx.x;
    const int per = tiles / 8;
    if (t < 8 * per) t = (t % 8) * per + t / 8;
    const int tm = t % p.tiles_m, tn = t / p.tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;

    const uint16_t* __restrict__ A = p.A + (int64_t)blockIdx.z * p.sA;
    const uint16_t* __restrict__ B = p.B + (int64_t)blockIdx.z * p.sB;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int K = p.K;
    const int nk = (K + BK - 1) / BK;
    // the last stage needs the guarded path when it reaches past K (A) or past
    // B's zero-padded width
    const bool tail_a = (nk * BK > K);
    const bool tail_b = (nk * BK > p.kread_b);

    auto issue = [&](int kt) {
        uint16_t* slot = smem + (kt % STAGES) * SLOT;
        const int k0 = kt * BK;
        const bool last = (kt == nk - 1);
        if (last && tail_a) stage_guarded<BM, NW>(A, p.lda, m0, p.M - 1, k0, K, slot, wave, lane);
        else stage_direct<BM, NW>(A, p.lda, m0, p.M - 1, k0, slot, wave, lane);
        if (last && tail_b) stage_guarded<BN, NW>(B, p.ldb, n0, p.N - 1, k0, p.kread_b, slot + BM * ROWH, wave, lane);
        else stage_direct<BN, NW>(B, p.ldb, n0, p.N - 1, k0, slot + BM * ROWH, wave, lane);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Fragment reads of k-step ks of the stage held in ring slot `slot_idx`.
    // They are inline-asm LDS reads with explicit waits (device_math.h): the
    // compiler's own waits would put vmcnt(0) before every read (the ring is
    // filled by direct loads) and merge the loop-carried reads into
    // lgkmcnt(0).  Row r of a fragment is lane&31 plus a multiple of 32, so its
    // swizzle (r >> 1) & 7 is the lane's; byte offsets: row * 128 + slot * 16.
    struct Frags { u32x4 a[TM]; u32x4 b[TN]; };
    const uint32_t lds0 = lds_offset(smem);
    const uint32_t a_lane = (uint32_t)((wm * WM + (lane & 31)) * ROWH * 2);
    const uint32_t b_lane = (uint32_t)((BM + wn * WN + (lane & 31)) * ROWH * 2);
    const int swz = (lane >> 1) & 7, half = lane >> 5;
    auto load_frags = [&](int slot_idx, int ks, Frags& f) {
        const uint32_t base = lds0 + (uint32_t)(slot_idx * SLOT * 2) + (uint32_t)((((2 * ks + half) ^ swz)) << 4);
#pragma unroll
        for (int i = 0; i < TM; ++i) f.a[i] = asm_lds_read_b128(base + a_lane + i * 32 * ROWH * 2);
#pragma unroll
        for (int j = 0; j < TN; ++j) f.b[j] = asm_lds_read_b128(base + b_lane + j * 32 * ROWH * 2);
    };
    // wait until at most `newer` LDS reads are pending, then tie f to the wait
    auto ready = [&](Frags& f, bool newer) {
        if (newer) asm_wait_lgkmcnt<TM + TN>();
        else asm_wait_lgkmcnt<0>();
#pragma unroll
        for (int i = 0; i < TM; ++i) asm_pin(f.a[i]);
#pragma unroll
        for (int j = 0; j < TN; ++j) asm_pin(f.b[j]);
    };
    auto mma = [&](const Frags& f) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = mfma32<BF16>(f.a[i], f.b[j], acc[i][j]);
    };
    // Stage s has landed in LDS for every wave once this returns.  `later`
    // stages were issued after s; those issued by the direct path may stay in
    // flight (vmcnt counts them in issue order).
    auto wait_stage = [&](int s, int later) {
        const int later_direct = later - ((later > 0 && s + later == nk - 1 && (tail_a || tail_b)) ? 1 : 0);
        if (later_direct >= 2) asm_wait_vmcnt<(2 * LA <= 63) ? 2 * LA : LA>();   // LA: conservative
        else if (later_direct == 1) asm_wait_vmcnt<LA>();
        else asm_wait_vmcnt<0>();
        // A bare s_barrier, not __syncthreads(): the latter's release fence
        // would wait for every in-flight stage (vmcnt(0)).  LDS traffic (this
        // wave's last fragment reads of the slot about to be refilled, and the
        // guarded stage's ds_writes) is drained first.
        asm_wait_lgkmcnt<0>();
        __builtin_amdgcn_s_barrier();
    };

#pragma unroll
    for (int s = 0; s < STAGES; ++s)
        if (s < nk) issue(s);
    wait_stage(0, min(STAGES, nk) - 1);

    // Main loop.  Fragments are double-buffered: the reads of k-step ks+1 are
    // issued before the MFMAs of k-step ks.  Before the last k-step's MFMAs the
    // wave waits for the next stage and meets the others at the barrier, then
    // refills the current slot with stage kt+STAGES (its last reads, k-step 3,
    // were issued during k-step 2 and drained before the barrier) and reads the
    // next stage's first fragments, so neither the barrier nor that read sits
    // in front of an idle matrix core.  Stage kt+1 was issued STAGES-1
    // iterations before it is waited for.
    // Two fragment sets alternate by k-step parity (BK/16 = 4 k-steps per
    // stage, so a stage always starts on set 0); with the k-step loop unrolled
    // they are distinct registers and no copies are needed.
    Frags f[2];
    load_frags(0, 0, f[0]);
    for (int kt = 0; kt < nk; ++kt) {
        const int slot_idx = kt % STAGES;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            Frags& nxt = f[(ks + 1) & 1];
            if (ks < BK / 16 - 1) {
                load_frags(slot_idx, ks + 1, nxt);
            } else if (kt + 1 < nk) {
                wait_stage(kt + 1, min(kt + STAGES - 1, nk - 1) - (kt + 1));
                if (kt + STAGES < nk) issue(kt + STAGES);
                load_frags((kt + 1) % STAGES, 0, nxt);
            }
            // LDS reads complete in order: with the TM+TN reads of the next set
            // issued last, lgkmcnt(TM+TN) means this set has landed.  (At the
            // last k-step of the last stage nothing newer is pending.)
            ready(f[ks & 1], ks < BK / 16 - 1 || kt + 1 < nk);
            mma(f[ks & 1]);
        }
    }

    const int64_t c_off = (int64_t)blockIdx.z * p.sC;
    if (!p.ep_on) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = n0 + wn * WN + j * 32 + (lane & 31);
                if (col >= p.N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row < p.M) store_out(p.C, c_off + (int64_t)row * p.ldc + col, acc[i][j][r], p.c_dtype);
                }
            }
    } else {   // fused epilogue: the per-element code is larger, so only the tile loops unroll
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = n0 + wn * WN + j * 32 + (lane & 31);
                if (col >= p.N) continue;
#pragma unroll 4
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (row < p.M) {
                        const int64_t idx = c_off + (int64_t)row * p.ldc + col;
                        store_out(p.C, idx, apply_epilogue(p.ep, acc[i][j][r], idx, col), p.c_dtype);
                    }
                }
            }
    }
}

// ---- launch configuration ----------------------------------------------------

typedef void (*GemmKernel)(const GemmArgs);

struct TileCfg {
    int bm, bn, stages, waves;
    int per_cu;       // resident blocks per CU (LDS ring and registers)
    int eff;          // TFLOP/s of a full-wave 4096^3 fp16 run (selection weight)
    GemmKernel f16, bf16;
};

#define MVLM_TILE(BMv, BNv, Sv, WMv, WNv, PER_CU, EFF)                                             \
    TileCfg{BMv, BNv, Sv, WMv * WNv, PER_CU, EFF, gemm_mfma_kernel<false, BMv, BNv, Sv, WMv, WNv>, \
            gemm_mfma_kernel<true, BMv, BNv, Sv, WMv, WNv>}
// The first four are the automatic choices; the others are kept for tuning.
static const TileCfg kTiles[] = {
    MVLM_TILE(256, 256, 2, 4, 2, 1, 831), MVLM_TILE(256, 128, 2, 4, 2, 1, 714),
    MVLM_TILE(128, 128, 4, 4, 2, 1, 537), MVLM_TILE(64, 64, 4, 2, 2, 2, 386),
    MVLM_TILE(256, 128, 3, 4, 2, 1, 628), MVLM_TILE(128, 128, 4, 2, 2, 1, 502),
    MVLM_TILE(128, 64, 4, 2, 2, 1, 375),
};
constexpr int kAutoTiles = 4;
#undef MVLM_TILE

// The tile with the best (full-wave throughput x fraction of the last round
// of blocks that is busy x fraction of computed outputs that are stored).
// MVLM_GEMM_TILE=<bm>x<bn>s<stages>w<waves> forces a compiled tile (tuning runs).
static const TileCfg& pick_tile(int M, int N, int batch, int num_cus) {
    static const char* force = std::getenv("MVLM_GEMM_TILE");
    if (force) {
        int bm = 0, bn = 0, st = 0, w = 0;
        if (std::sscanf(force, "%dx%ds%dw%d", &bm, &bn, &st, &w) == 4)
            for (const TileCfg& c : kTiles)
                if (c.bm == bm && c.bn == bn && c.stages == st && c.waves == w) return c;
    }
    const TileCfg* best = &kTiles[kAutoTiles - 1];
    double best_score = -1.0;
    for (int i = 0; i < kAutoTiles; ++i) {
        const TileCfg& c = kTiles[i];
        const int64_t tiles = (int64_t)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * batch;
        const int64_t slots = (int64_t)num_cus * c.per_cu;
        const int64_t rounds = (tiles + slots - 1) / slots;
        const double fill = (double)tiles / (double)(rounds * slots);
        const double useful = (double)M * N * batch / (double)(tiles * c.bm * c.bn);
        const double score = c.eff * fill * useful;
        if (score > best_score) { best_score = score; best = &c; }
    }
    return *best;
}

hipError_t launch_gemm_mfma(hipStream_t s, const void* A, int ab_dtype, const void* B, void* C, int c_dtype,
                            int batch, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
                            int64_t strideA, int64_t strideB, int64_t strideC, int kread_b, int num_cus,
                            const Epilogue* ep) {
    GemmArgs a{};
    a.A = (const uint16_t*)A; a.B = (const uint16_t*)B; a.C = C; a.c_dtype = c_dtype;
    a.M = M; a.N = N; a.K = K; a.lda = lda; a.ldb = ldb; a.ldc = ldc;
    a.sA = strideA; a.sB = strideB; a.sC = strideC;
    a.kread_b = kread_b;
    if (ep && ep->any()) {
        a.ep = *ep;
        a.ep_on = 1;
    }
    const TileCfg& t = pick_tile(M, N, batch, num_cus > 0 ? num_cus : 256);
    a.tiles_m = (M + t.bm - 1) / t.bm;
    a.tiles_n = (N + t.bn - 1) / t.bn;
    dim3 grid((unsigned)(a.tiles_m * a.tiles_n), 1, (unsigned)batch);
    launch_kernel(ab_dtype == MVLM_BF16 ? t.bf16 : t.f16, grid, dim3(64 * t.waves), 0, s, a);
    return hipGetLastError();
}

}  // namespace mvlm
