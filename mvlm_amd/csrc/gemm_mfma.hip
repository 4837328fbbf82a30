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
//  * global -> LDS with direct 16-byte loads (buffer_load_dwordx4 ... lds
//    through a descriptor over the tile's rows on the large tiles,
//    global_load_lds_dwordx4 on the others): one wave instruction moves
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
#include <type_traits>

namespace mvlm {

// LDS geometry of a stage BK elements wide: one row per operand row, RB bytes
// (LPR 16-byte slots); one direct-load instruction fills RPI rows (1 KiB).
// Slot s of row r is stored at s ^ swz(r): a ds_read_b128 phase (16 lanes,
// 16 consecutive rows, one logical slot) then hits 16 distinct 16-byte bank
// groups of the 256-byte bank period (one 256-byte row, two 128-byte rows, or
// four 64-byte rows).
template <int BK>
struct StageGeom {
    static_assert(BK == 32 || BK == 64 || BK == 128, "stage width");
    static constexpr int ROWH = BK, RB = 2 * BK, LPR = RB / 16, RPI = 1024 / RB;
    __device__ static __forceinline__ int swz(int r) {
        return BK == 128 ? r & 15 : BK == 64 ? (r >> 1) & 7 : (r >> 2) & 3;
    }
};

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
    // split-K: grid z = batch * splits; split s covers K stages
    // [s * split_stages, (s + 1) * split_stages) and, when splits > 1, writes
    // its fp32 partial to ws[(b * splits + s) * M * N + m * N + n] for
    // gemm_splitk_reduce_kernel (which then applies the epilogue)
    int splits, split_stages;
    float* ws;
    // 4 consecutive columns of a row start 16-byte (fp32) / 8-byte (16-bit)
    // aligned in C (vec_c) and in the split partials (vec_ws), so one vector
    // store writes them
    int vec_c, vec_ws;
};

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{})
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// fp32 partial of 4 consecutive columns (n_left of them below N; the row
// starts 16-byte aligned)
__device__ __forceinline__ void store_partial4(float* ws, int64_t i, f32x4 v, int n_left) {
    if (n_left >= 4) {
        asm_global_store_b128_wt(ws + i, __builtin_bit_cast(u32x4, v));
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (e < n_left) ws[i + e] = v[e];
}

// C row `row_off` (element offset of the row), columns col..col+3: epilogue,
// output dtype, one 16- or 8-byte store when the row is aligned for it,
// written through L2 (C is tens of MB at the prefill shapes)
__device__ __forceinline__ void store_c4(const GemmArgs& p, int64_t row_off, int col, f32x4 v) {
    const int n_left = p.N - col;
    if (n_left <= 0) return;
    if (p.ep_on) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t idx = row_off + col + e;
            if (e < n_left) v[e] = apply_epilogue(p.ep, v[e], idx, col + e);
        }
    }
    const int64_t i = row_off + col;
    if (p.vec_c && n_left >= 4) {
        if (p.c_dtype == 0) {
            asm_global_store_b128_wt((float*)p.C + i, __builtin_bit_cast(u32x4, v));
        } else {
            u32x2 h;
            if (p.c_dtype == 1) {
                h[0] = f32_to_f16_bits(v[0]) | ((uint32_t)f32_to_f16_bits(v[1]) << 16);
                h[1] = f32_to_f16_bits(v[2]) | ((uint32_t)f32_to_f16_bits(v[3]) << 16);
            } else {
                h[0] = f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
                h[1] = f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
            }
            asm_global_store_b64_wt((uint16_t*)p.C + i, h);
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (e < n_left) store_out(p.C, i + e, v[e], p.c_dtype);
}

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    if constexpr (BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Direct loads of one operand's stage: ROWS rows starting at tile row r0,
// K columns [k0, k0+BK).  Wave w of NW issues RPI-row groups w, w+NW, ...;
// lane i writes LDS bytes [16i, 16i+16) of its group, i.e. row RPI g + i/LPR,
// physical slot i%LPR, and so fetches logical slot (i%LPR) ^ swz(row).
template <int BK, int ROWS, int NW>
__device__ __forceinline__ void stage_direct(const uint16_t* __restrict__ base, int64_t ld, int r0, int rmax, int k0,
                                             uint16_t* lds, int wave, int lane) {
    using G = StageGeom<BK>;
    static_assert((ROWS / G::RPI) % NW == 0, "row groups must split evenly over the waves");
#pragma unroll
    for (int t = 0; t < ROWS / (G::RPI * NW); ++t) {
        const int g = wave + NW * t;
        const int lr = G::RPI * g + lane / G::LPR;
        const int ls = (lane % G::LPR) ^ G::swz(lr);
        const int r = min(r0 + lr, rmax);
        const uint16_t* src = base + (int64_t)r * ld + k0 + ls * 8;
        asm_global_load_lds_b128(src, __builtin_amdgcn_readfirstlane(lds_offset(lds + G::RPI * g * G::ROWH)));
    }
}

// stage_direct through a buffer descriptor whose base is the tile's first row:
// a 32-bit offset per lane instead of a 64-bit address (fewer VGPRs, and the
// Phi-1.5 M = 768 shapes and 4096^3 2-5% faster; the SigLIP tiles keep the
// global form, which measured as fast or faster there)
template <int BK, int ROWS, int NW>
__device__ __forceinline__ void stage_direct_buf(i32x4 rsrc, int64_t ld, int r0, int rmax, int k0, uint16_t* lds,
                                                 int wave, int lane) {
    using G = StageGeom<BK>;
    static_assert((ROWS / G::RPI) % NW == 0, "row groups must split evenly over the waves");
#pragma unroll
    for (int t = 0; t < ROWS / (G::RPI * NW); ++t) {
        const int g = wave + NW * t;
        const int lr = G::RPI * g + lane / G::LPR;
        const int ls = (lane % G::LPR) ^ G::swz(lr);
        const int r = min(r0 + lr, rmax) - r0;
        const uint32_t off = (uint32_t)(((int64_t)r * ld + k0 + ls * 8) * 2);
        asm_buffer_load_lds_b128(rsrc, off, __builtin_amdgcn_readfirstlane(lds_offset(lds + G::RPI * g * G::ROWH)));
    }
}

// Guarded loads of the last stage: 16-byte chunks at or beyond kread are zero.
template <int BK, int ROWS, int NW>
__device__ __forceinline__ void stage_guarded(const uint16_t* __restrict__ base, int64_t ld, int r0, int rmax, int k0,
                                              int kread, uint16_t* lds, int wave, int lane) {
    using G = StageGeom<BK>;
    static_assert((ROWS / G::RPI) % NW == 0, "row groups must split evenly over the waves");
#pragma unroll
    for (int t = 0; t < ROWS / (G::RPI * NW); ++t) {
        const int g = wave + NW * t;
        const int lr = G::RPI * g + lane / G::LPR;
        const int ls = (lane % G::LPR) ^ G::swz(lr);
        const int r = min(r0 + lr, rmax);
        const int k = k0 + ls * 8;
        u32x4 v = {0, 0, 0, 0};
        if (k < kread) v = *reinterpret_cast<const u32x4*>(base + (int64_t)r * ld + k);
        *reinterpret_cast<u32x4*>(lds + G::RPI * g * G::ROWH + lane * 8) = v;
    }
}

template <bool BF16, int BM, int BN, int BK, int STAGES, int WGM, int WGN, bool BUF>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_mfma_kernel(const GemmArgs p) {
    using G = StageGeom<BK>;
    constexpr int ROWH = G::ROWH;
    constexpr int NW = WGM * WGN;                // waves per block (WGM x WGN grid)
    constexpr int WM = BM / WGM, WN = BN / WGN;  // wave sub-tile
    constexpr int TM = WM / 32, TN = WN / 32;    // 32x32 MFMA tiles per wave
    constexpr int LA = (BM + BN) / G::RPI / NW;  // direct-load instructions per wave per stage
    constexpr int SLOT = (BM + BN) * ROWH;       // elements per ring slot
    static_assert(TM + TN <= 15, "fragment reads must fit the lgkmcnt field");
    // the store pass reuses the ring: a 32 x 36 fp32 staging tile per wave
    static_assert(STAGES * SLOT * 2 >= NW * 32 * 36 * 4, "ring too small for the store staging");
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

    const int batch = blockIdx.z / p.splits, split = blockIdx.z % p.splits;
    const uint16_t* __restrict__ A = p.A + (int64_t)batch * p.sA;
    const uint16_t* __restrict__ B = p.B + (int64_t)batch * p.sB;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int K = p.K;
    const int nk_all = (K + BK - 1) / BK;
    const int kt0 = split * p.split_stages;                     // this split's first stage
    const int nk = min(nk_all - kt0, p.split_stages);           // stages of this split (>= 1)
    // the global last stage needs the guarded path when it reaches past K (A)
    // or past B's zero-padded width
    const bool tail_a = (nk_all * BK > K) && kt0 + nk == nk_all;
    const bool tail_b = (nk_all * BK > p.kread_b) && kt0 + nk == nk_all;

    // BUF: descriptors over the tile's rows of A and B (every offset stays below
    // the 32-bit size, checked by the launcher)
    const i32x4 ra = raw_rsrc(A + (int64_t)m0 * p.lda, BUF ? (uint32_t)((int64_t)(p.M - m0) * p.lda * 2) : 0u);
    const i32x4 rb = raw_rsrc(B + (int64_t)n0 * p.ldb, BUF ? (uint32_t)((int64_t)(p.N - n0) * p.ldb * 2) : 0u);
    auto issue = [&](int kt) {
        uint16_t* slot = smem + (kt % STAGES) * SLOT;
        const int k0 = (kt0 + kt) * BK;
        const bool last = (kt == nk - 1);
        if (last && tail_a) stage_guarded<BK, BM, NW>(A, p.lda, m0, p.M - 1, k0, K, slot, wave, lane);
        else if constexpr (BUF) stage_direct_buf<BK, BM, NW>(ra, p.lda, m0, p.M - 1, k0, slot, wave, lane);
        else stage_direct<BK, BM, NW>(A, p.lda, m0, p.M - 1, k0, slot, wave, lane);
        if (last && tail_b)
            stage_guarded<BK, BN, NW>(B, p.ldb, n0, p.N - 1, k0, p.kread_b, slot + BM * ROWH, wave, lane);
        else if constexpr (BUF) stage_direct_buf<BK, BN, NW>(rb, p.ldb, n0, p.N - 1, k0, slot + BM * ROWH, wave, lane);
        else stage_direct<BK, BN, NW>(B, p.ldb, n0, p.N - 1, k0, slot + BM * ROWH, wave, lane);
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
    // swizzle is the lane's; byte offsets: row * RB + slot * 16.
    struct Frags { u32x4 a[TM]; u32x4 b[TN]; };
    const uint32_t lds0 = lds_offset(smem);
    const uint32_t a_lane = (uint32_t)((wm * WM + (lane & 31)) * ROWH * 2);
    const uint32_t b_lane = (uint32_t)((BM + wn * WN + (lane & 31)) * ROWH * 2);
    const int swz = G::swz(lane & 31), half = lane >> 5;
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
    // Two fragment sets alternate by k-step parity (BK/16 = 4 or 2 k-steps per
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

    const int64_t c_off = (int64_t)batch * p.sC;
    float* ws = p.splits > 1 ? p.ws + (int64_t)blockIdx.z * p.M * p.N : nullptr;
    const bool vec = ws ? p.vec_ws : p.vec_c;
    if (!vec) {   // rows off the vector grid: straight from the accumulators, 32 columns per row
        if (ws) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const int col = n0 + wn * WN + j * 32 + (lane & 31);
                    if (col >= p.N) continue;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        if (row < p.M) ws[(int64_t)row * p.N + col] = acc[i][j][r];
                    }
                }
        } else if (!p.ep_on) {
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
        return;
    }
    // Aligned rows: through LDS.  Each wave writes one 32x32 accumulator tile
    // at a time into its own region of the (now idle) ring, row-major with a
    // 36-float pitch (rows r and r+4, written by lanes l and l+32, land 16
    // banks apart), and reads it back as 4 consecutive columns per lane, 8 rows
    // per pass: 16-byte global stores, and per-element code (epilogue, dtype)
    // in a loop rather than unrolled over the 16 * TM * TN accumulators.
    __syncthreads();   // every wave is done with the ring (all its loads have landed)
    constexpr int CS = 36;
    float* cst = reinterpret_cast<float*>(smem) + wave * 32 * CS;
    const int srow = lane >> 3, scol = (lane & 7) * 4;
    // (compile-time tile indices: a rolled tile loop would index acc at run time
    // and move it to scratch memory)
    static_for<TM * TN>([&](auto IJ) {
        constexpr int i = decltype(IJ)::value / TN, j = decltype(IJ)::value % TN;
        {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                cst[(8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * CS + (lane & 31)] = acc[i][j][r];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's writes, before its reads
            const int row0 = m0 + wm * WM + i * 32, col = n0 + wn * WN + j * 32 + scol;
            for (int t = 0; t < 4; ++t) {
                const int row = row0 + srow + 8 * t;
                const f32x4 v = *reinterpret_cast<const f32x4*>(cst + (srow + 8 * t) * CS + scol);
                if (row >= p.M) continue;
                if (ws) store_partial4(ws, (int64_t)row * p.N + col, v, p.N - col);
                else store_c4(p, c_off + (int64_t)row * p.ldc, col, v);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // reads done before the next tile's writes
        }
    });
}

// Sums the split-K partials in split order (deterministic), applies the
// epilogue and stores C: thread = V consecutive output elements of the
// flattened [M][N] (V = 4 reads the partials as 16-byte vectors; it needs
// M*N % 4 == 0 so every split's partial stays 16-byte aligned).
template <int V>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const GemmArgs p) {
    const int64_t mn = (int64_t)p.M * p.N;
    const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
    const int b = blockIdx.y;
    if (i0 >= mn) return;
    const float* ws = p.ws + (int64_t)b * p.splits * mn + i0;
    float v[V];
    if constexpr (V == 4) {
        f32x4 acc = *reinterpret_cast<const f32x4*>(ws);
        for (int s = 1; s < p.splits; ++s) acc += *reinterpret_cast<const f32x4*>(ws + s * mn);
        v[0] = acc[0]; v[1] = acc[1]; v[2] = acc[2]; v[3] = acc[3];
    } else {
        v[0] = 0.0f;
        for (int s = 0; s < p.splits; ++s) v[0] += ws[s * mn];
    }
    if constexpr (V == 4) {
        // N % 4 == 0: the four elements share a row, and with vec_c they are
        // one aligned 16-byte (fp32) or 8-byte (16-bit) piece of C
        if (p.vec_c && p.N % 4 == 0) {
            const int row = (int)(i0 / p.N), col = (int)(i0 - (int64_t)row * p.N);
            const int64_t idx = (int64_t)b * p.sC + (int64_t)row * p.ldc + col;
            store_c4(p, idx - col, col, (f32x4){v[0], v[1], v[2], v[3]});
            return;
        }
    }
#pragma unroll
    for (int e = 0; e < V; ++e) {
        const int64_t i = i0 + e;
        const int row = (int)(i / p.N), col = (int)(i - (int64_t)row * p.N);
        const int64_t idx = (int64_t)b * p.sC + (int64_t)row * p.ldc + col;
        store_out(p.C, idx, p.ep_on ? apply_epilogue(p.ep, v[e], idx, col) : v[e], p.c_dtype);
    }
}

// ---- launch configuration ----------------------------------------------------

typedef void (*GemmKernel)(const GemmArgs);

struct TileCfg {
    int bm, bn, bk, stages, waves;
    int per_cu;       // resident blocks per CU (LDS ring and registers)
    int eff;          // TFLOP/s of a full-wave 4096^3 fp16 run (selection weight)
    bool buf;         // buffer-addressed direct loads: operands below 4 GiB only
    GemmKernel f16, bf16;
};

#define MVLM_TILE_X(BMv, BNv, BKv, Sv, WMv, WNv, PER_CU, EFF, BUFv)                                         \
    TileCfg{BMv, BNv, BKv, Sv, WMv * WNv, PER_CU, EFF, BUFv, gemm_mfma_kernel<false, BMv, BNv, BKv, Sv, WMv, WNv, BUFv>, \
            gemm_mfma_kernel<true, BMv, BNv, BKv, Sv, WMv, WNv, BUFv>}
#define MVLM_TILE(BMv, BNv, BKv, Sv, WMv, WNv, PER_CU, EFF) MVLM_TILE_X(BMv, BNv, BKv, Sv, WMv, WNv, PER_CU, EFF, false)
#define MVLM_TILE_B(BMv, BNv, BKv, Sv, WMv, WNv, PER_CU, EFF) MVLM_TILE_X(BMv, BNv, BKv, Sv, WMv, WNv, PER_CU, EFF, true)
// The first nine are the automatic choices (eff measured at 4096^3, fp16 in,
// fp32 out); the others are kept for tuning.  The 128-wide stages halve a
// block's stage count (and its waits and barriers), which pays on the short-K
// SigLIP shapes (729 x 1152 x 1152: 11.4 -> 9.4 us with 64 x 64 tiles; 729 x
// 4304 x 1152: 18.7 -> 16.9 us with 128 x 128) and, as two 80 KiB stages of
// 192 x 128, a little on 768-row shapes (~1%) and 1536 x 6144 x 2048 (73.3 ->
// 70.1 us); the 64-wide 64 x 64 tile stays for the many-way K splits of
// few-row products.  96 x 192 with six waves of 32 x 96 cuts 768 x 6144 into
// exactly 256 blocks (192 with 192 x 128): 35.4 -> 34.3 us at that shape.
static const TileCfg kTiles[] = {
    MVLM_TILE_B(256, 256, 64, 2, 4, 2, 1, 907), MVLM_TILE_B(256, 128, 64, 2, 4, 2, 1, 785),
    MVLM_TILE_B(192, 128, 64, 3, 2, 4, 1, 636), MVLM_TILE(128, 128, 64, 4, 4, 2, 1, 619),
    MVLM_TILE(64, 64, 64, 4, 2, 2, 2, 401), MVLM_TILE(128, 128, 128, 2, 4, 2, 1, 682),
    MVLM_TILE(64, 64, 128, 2, 2, 2, 2, 460), MVLM_TILE_B(192, 128, 128, 2, 2, 4, 1, 700),
    MVLM_TILE_B(96, 192, 128, 2, 3, 2, 1, 564),
    MVLM_TILE(256, 128, 64, 3, 4, 2, 1, 628), MVLM_TILE(128, 128, 64, 4, 2, 2, 1, 502),
    MVLM_TILE(128, 64, 64, 4, 2, 2, 1, 375),
    MVLM_TILE(256, 256, 32, 4, 4, 2, 1, 849), MVLM_TILE(256, 256, 32, 5, 4, 2, 1, 828),
    MVLM_TILE(256, 128, 32, 6, 4, 2, 1, 686), MVLM_TILE(128, 128, 32, 8, 4, 2, 1, 541),
    MVLM_TILE(128, 128, 32, 4, 4, 2, 2, 689), MVLM_TILE(192, 128, 32, 6, 2, 2, 1, 460),
};
constexpr int kAutoTiles = 9;
#undef MVLM_TILE
#undef MVLM_TILE_B
#undef MVLM_TILE_X

struct GemmPlan {
    const TileCfg* tile;
    int splits, split_stages;
};

// The tile and K split with the least modelled time: block rounds x one
// block's share of the tile's full-chip throughput (eff, all slots busy),
// plus, for a split, writing and re-reading the fp32 partials (~4 TB/s) and a
// second launch.  MVLM_GEMM_TILE=<bm>x<bn>s<stages>w<waves>[k<bk>] forces a
// compiled tile and MVLM_GEMM_SPLITS=<n> a split count (tuning runs; read at
// every launch).
static GemmPlan plan_gemm(int M, int N, int K, int batch, int num_cus, bool buf_ok) {
    GemmPlan best{&kTiles[4], 1, 0};
    double best_t = 1e30;
    const char* force = std::getenv("MVLM_GEMM_TILE");
    const TileCfg* forced = nullptr;
    if (force) {
        int bm = 0, bn = 0, st = 0, w = 0, bk = 64;
        if (std::sscanf(force, "%dx%ds%dw%dk%d", &bm, &bn, &st, &w, &bk) >= 4)
            for (const TileCfg& c : kTiles)
                if (c.bm == bm && c.bn == bn && c.stages == st && c.waves == w && c.bk == bk && (buf_ok || !c.buf))
                    forced = &c;
    }
    const char* fs = std::getenv("MVLM_GEMM_SPLITS");
    const int forced_splits = fs ? std::atoi(fs) : 0;
    // K <= 128 (e.g. attention scores, head_dim 72): a block's time is its load
    // latency and its C store, not its MFMAs, which the model above does not
    // see; 128x128 tiles with 32-wide stages (less K padding, two blocks per
    // CU) measured fastest there (16 x 729x729x72: 19.9 us vs 25.2 us).
    if (!forced && K <= 128 && forced_splits <= 1)
        for (const TileCfg& c : kTiles)
            if (c.bm == 128 && c.bn == 128 && c.bk == 32 && c.per_cu == 2) forced = &c;
    const int n_cand = forced ? 1 : kAutoTiles;
    for (int i = 0; i < n_cand; ++i) {
        const TileCfg& c = forced ? *forced : kTiles[i];
        if (c.buf && !buf_ok) continue;
        const int nk = (K + c.bk - 1) / c.bk;
        for (int splits : {1, 2, 3, 4, 6, 8}) {
            if (forced_splits > 0 && splits != forced_splits) continue;
            if (splits > 1 && nk < 4 * splits) break;                 // keep at least 4 stages per split
            const int ss = (nk + splits - 1) / splits;
            const int used = (nk + ss - 1) / ss;                         // non-empty splits
            if (used != splits) continue;
            const int64_t tiles = (int64_t)((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * batch * splits;
            const int64_t slots = (int64_t)num_cus * c.per_cu;
            const int64_t rounds = (tiles + slots - 1) / slots;
            const double block_flops = 2.0 * c.bm * c.bn * (double)ss * c.bk;
            const double eff = c.eff > 0 ? c.eff : 100.0;              // unmeasured tuning tiles
            double t = rounds * block_flops / (eff * 1e12 / (double)slots);
            if (splits > 1) t += (double)M * N * batch * 4.0 * (2.0 * splits + 1.0) / 4e12 + 3e-6;
            if (t < best_t) { best_t = t; best = GemmPlan{&c, splits, ss}; }
        }
    }
    if (best.split_stages == 0) best.split_stages = (K + best.tile->bk - 1) / best.tile->bk;
    return best;
}

// Copies rows of K elements (row r of batch b at src + b*stride + r*ld) into
// dst [batch][rows][Kp], zero-filling columns K..Kp-1.
__global__ __launch_bounds__(256) void gemm_pad_rows_kernel(const uint16_t* __restrict__ src, int64_t ld,
                                                            int64_t stride, int rows, int K, uint16_t* __restrict__ dst,
                                                            int Kp, int64_t total) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / Kp;
        const int k = (int)(i - r * Kp);
        const int64_t b = r / rows, rr = r - b * rows;
        dst[i] = k < K ? src[b * stride + rr * ld + k] : (uint16_t)0;
    }
}

// Workspace layout: [split partials][padded A][padded B], each 256-byte aligned.
struct GemmWorkspace {
    bool pad_a = false, pad_b = false;
    int kp = 0;                    // K the kernel runs with (zero columns past K)
    GemmPlan plan{};
    size_t split_bytes = 0, a_off = 0, b_off = 0, total = 0;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static GemmWorkspace gemm_workspace(int batch, int M, int N, int K, int64_t lda, int64_t ldb, int64_t sA,
                                   int64_t sB, int kread_b, int num_cus) {
    GemmWorkspace w;
    const int k8 = (int)round_up(K, 8);
    w.pad_a = K % 8 != 0 || lda % 8 != 0 || (batch > 1 && sA % 8 != 0);
    w.pad_b = ldb % 8 != 0 || (batch > 1 && sB % 8 != 0) || kread_b < k8;
    w.kp = (w.pad_a || w.pad_b) ? k8 : K;
    // buffer-addressed tiles need each operand's rows within a 32-bit byte range
    const int64_t lda_k = w.pad_a ? w.kp : lda, ldb_k = w.pad_b ? w.kp : ldb;
    const bool buf_ok = (int64_t)M * lda_k * 2 < ((int64_t)1 << 32) - 256 && (int64_t)N * ldb_k * 2 < ((int64_t)1 << 32) - 256;
    w.plan = plan_gemm(M, N, w.kp, batch, num_cus > 0 ? num_cus : 256, buf_ok);
    w.split_bytes = w.plan.splits > 1 ? align256((size_t)w.plan.splits * batch * M * N * sizeof(float)) : 0;
    w.a_off = w.split_bytes;
    const size_t a_bytes = w.pad_a ? align256((size_t)batch * M * w.kp * 2) : 0;
    w.b_off = w.a_off + a_bytes;
    const size_t b_bytes = w.pad_b ? align256((size_t)batch * N * w.kp * 2) : 0;
    w.total = w.b_off + b_bytes;
    return w;
}

size_t gemm_workspace_bytes(int batch, int M, int N, int K, int64_t lda, int64_t ldb, int64_t sA, int64_t sB,
                            int kread_b, int num_cus) {
    return gemm_workspace(batch, M, N, K, lda, ldb, sA, sB, kread_b, num_cus).total;
}

// Launches kernel `idx` of an op made of `n` kernels (plan profiling times the
// first kernel's start to the last one's stop).
template <typename... KArgs, typename... Args>
static void launch_seq(int idx, int n, void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t s,
                       Args&&... args) {
    if (n == 1) launch_kernel(kernel, grid, block, 0, s, std::forward<Args>(args)...);
    else launch_kernel_part(idx == 0 ? LaunchPart::First : idx == n - 1 ? LaunchPart::Last : LaunchPart::Middle,
                            kernel, grid, block, 0, s, std::forward<Args>(args)...);
}

static unsigned pad_grid(int64_t total) {
    const int64_t b = (total + 255) / 256;
    return (unsigned)(b < 4096 ? b : 4096);
}

hipError_t launch_gemm_mfma(hipStream_t s, const void* A, int ab_dtype, const void* B, void* C, int c_dtype,
                            int batch, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
                            int64_t strideA, int64_t strideB, int64_t strideC, int kread_b, int num_cus,
                            const Epilogue* ep, void* workspace, size_t workspace_bytes) {
    const GemmWorkspace w = gemm_workspace(batch, M, N, K, lda, ldb, strideA, strideB, kread_b, num_cus);
    if (w.total > 0 && (!workspace || workspace_bytes < w.total)) return hipErrorInvalidValue;
    const GemmPlan& g = w.plan;
    const TileCfg& t = *g.tile;
    GemmArgs a{};
    a.A = (const uint16_t*)A; a.B = (const uint16_t*)B; a.C = C; a.c_dtype = c_dtype;
    a.M = M; a.N = N; a.K = w.kp; a.lda = lda; a.ldb = ldb; a.ldc = ldc;
    a.sA = strideA; a.sB = strideB; a.sC = strideC;
    a.kread_b = kread_b;
    if (ep && ep->any()) {
        a.ep = *ep;
        a.ep_on = 1;
    }
    a.tiles_m = (M + t.bm - 1) / t.bm;
    a.tiles_n = (N + t.bn - 1) / t.bn;
    a.splits = g.splits;
    a.split_stages = g.split_stages;
    a.ws = (float*)workspace;
    {
        const int es = c_dtype == MVLM_F32 ? 4 : 2;
        a.vec_c = ((uintptr_t)C % (4 * es) == 0) && (ldc % 4 == 0) && (strideC % 4 == 0);
        a.vec_ws = N % 4 == 0;
    }
    const int n = (int)w.pad_a + (int)w.pad_b + 1 + (g.splits > 1 ? 1 : 0);
    int idx = 0;
    if (w.pad_a) {
        uint16_t* ap = (uint16_t*)((char*)workspace + w.a_off);
        const int64_t total = (int64_t)batch * M * w.kp;
        launch_seq(idx++, n, gemm_pad_rows_kernel, dim3(pad_grid(total)), dim3(256), s, (const uint16_t*)A, lda,
                   strideA, M, K, ap, w.kp, total);
        a.A = ap; a.lda = w.kp; a.sA = (int64_t)M * w.kp;
    }
    if (w.pad_b) {
        uint16_t* bp = (uint16_t*)((char*)workspace + w.b_off);
        const int64_t total = (int64_t)batch * N * w.kp;
        launch_seq(idx++, n, gemm_pad_rows_kernel, dim3(pad_grid(total)), dim3(256), s, (const uint16_t*)B, ldb,
                   strideB, N, min(K, kread_b), bp, w.kp, total);
        a.B = bp; a.ldb = w.kp; a.sB = (int64_t)N * w.kp; a.kread_b = w.kp;
    }
    dim3 grid((unsigned)(a.tiles_m * a.tiles_n), 1, (unsigned)(batch * g.splits));
    GemmKernel k = ab_dtype == MVLM_BF16 ? t.bf16 : t.f16;
    launch_seq(idx++, n, k, grid, dim3(64 * t.waves), s, a);
    if (g.splits > 1) {
        const int64_t mn = (int64_t)M * N;
        if (mn % 4 == 0)
            launch_seq(idx++, n, gemm_splitk_reduce_kernel<4>, dim3((unsigned)((mn / 4 + 255) / 256), (unsigned)batch),
                       dim3(256), s, a);
        else
            launch_seq(idx++, n, gemm_splitk_reduce_kernel<1>, dim3((unsigned)((mn + 255) / 256), (unsigned)batch),
                       dim3(256), s, a);
    }
    return hipGetLastError();
}

}  // namespace mvlm
