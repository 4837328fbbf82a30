// Per-chunk arithmetic and LDS staging of the streaming GEMV (gemv_stream.hip).
// A "chunk" is one 16-byte vector per lane, 1 KiB per wave, of one weight row:
// 4 fp32, 8 fp16/bf16, 16 Q8_0 codes (half a block) or 32 Q4_0 codes (one
// block) per lane.  Codes become fp32 in registers: v_cvt_f32_i32 with a byte
// select for Q8_0, masked nibbles through v_cvt_f32_ubyte* for Q4_0.  The block
// scale is applied once per half block (Q8_0) or block (Q4_0):
//   Q8_0: acc += d * sum_j x_j q_j
//   Q4_0: acc += d * (sum_j x_j c_j - 8 sum_j x_j),  c_j the 4-bit code.
// This is the GGUF dequantization (w = d*q, w = (c-8)*d) with d factored out
// of each block: different rounding, same value within the fp32 tolerance.
#pragma once

#include "common.h"
#include "device_math.h"

namespace mvlm {

// ---- weight formats --------------------------------------------------------

template <typename WT>
struct DenseFmt {
    static constexpr int WPL = 16 / (int)sizeof(WT);   // weights per lane per chunk
    static constexpr bool QUANT = false;
    static constexpr int MIN_WAVES_BATCH = 4;          // (dense weights take M = 1 only)
    static constexpr int MIN_WAVES = 8;                // per SIMD: 4 blocks of 8 waves per CU
};

struct Q8Fmt {
    static constexpr int WPL = 16;
    static constexpr bool QUANT = true;
    static constexpr int MIN_WAVES = 8;
    static constexpr int MIN_WAVES_BATCH = 4;          // 4 rows of x
};

struct Q4Fmt {
    static constexpr int WPL = 32;
    static constexpr bool QUANT = true;
    static constexpr int MIN_WAVES = 4;                // 32 x values per lane need more registers
    // 4 rows of x: at most 128 VGPRs (a few prologue values spill), so two
    // 8-wave blocks fit per CU; with 145 VGPRs only one did (M=4 step 568 -> 520 us)
    static constexpr int MIN_WAVES_BATCH = 4;
};

// x values of one chunk as raw bits: E elements of XT in XD dwords.
template <typename XT, int E>
struct XRaw {
    static constexpr int XD = E * (int)sizeof(XT) / 4;
    uint32_t d[XD];
};

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

// sum of the 32 x values of one Q4_0 block, in element order
template <typename XT, int E>
__device__ __forceinline__ float x_block_sum(const XRaw<XT, E>& xr) {
    float sx = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) sx += x_at(xr, j);
    return sx;
}

// byte j of the block holds weight j (low nibble) and weight j + 16 (high
// nibble); sx is the block's x_block_sum
template <typename XT, int E>
__device__ __forceinline__ float chunk_dot_q4(u32x4 q, uint16_t dh, const XRaw<XT, E>& xr, float sx, float acc) {
    float s = 0.0f;
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
    return __builtin_fmaf(f16_bits_to_f32(dh), __builtin_fmaf(-8.0f, sx, s), acc);
}

template <typename XT, int E>
__device__ __forceinline__ float chunk_dot(Q4Fmt, u32x4 q, uint16_t dh, const XRaw<XT, E>& xr, float acc) {
    return chunk_dot_q4(q, dh, xr, x_block_sum(xr), acc);
}


// ---- LDS staging -------------------------------------------------------------

// A lane's x values for one chunk are XB = WPL * sizeof(XT) consecutive bytes
// (8 .. 128).  Read from LDS as 16-byte slots, lane l reads slot SL*l + i in
// its i-th read; 16 lanes share one LDS cycle, so with SL > 1 lanes l and
// l + 16/SL would hit the same banks.  x is therefore stored with its 16-byte
// slot s at s ^ ((s >> 4) & (SL - 1)) (a permutation inside each 256-byte
// group, its own inverse), which gives the 16 lanes of a read 16 distinct
// bank groups.
template <int SL>
__device__ __forceinline__ int x_slot(int s) { return s ^ ((s >> 4) & (SL - 1)); }

// Copy nbytes (a multiple of W = 4 or 16) from global src into LDS dst with
// direct W-byte loads; the waves of the block take pieces of 64*W bytes in
// turn.  With SL > 1 the 16-byte slots are permuted by x_slot.  Source reads
// are clamped to [0, nbytes - W]: bytes landing beyond nbytes are never read,
// and the LDS region is rounded up to whole pieces.  CPOL is the loads' cache
// policy: 0, or kCpolDevice for data another workgroup of the same launch
// wrote with device-scope stores (read at the device coherence point, not from
// a possibly stale line of this XCD's L2).
constexpr int kCpolDevice = 16;   // sc1
template <int W, int SL, int NW, int CPOL = 0>
__device__ __forceinline__ void stage_to_lds(uint8_t* dst, const uint8_t* __restrict__ src, int nbytes,
                                             int wave, int lane) {
    static_assert(W == 4 || W == 16, "direct load width");
    for (int piece = wave; piece * 64 * W < nbytes; piece += NW) {
        const int phys = piece * 64 * W + lane * W;
        const int logical = x_slot<SL>(phys >> 4) * 16 + (phys & 15);
        const uint8_t* from = src + min(logical, nbytes - W);
        if constexpr (W == 16) __builtin_amdgcn_global_load_lds(from, (lds_void*)(dst + piece * 64 * W), 16, 0, CPOL);
        else __builtin_amdgcn_global_load_lds(from, (lds_void*)(dst + piece * 64 * W), 4, 0, CPOL);
    }
}

}  // namespace mvlm
