// Device-side number-format helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <cstdint>

namespace mvlm {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// v_cvt_f16_f32 rounds to nearest even under the default mode.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

// Widen the raw 16-bit pattern of an fp16 / bf16 element.
template <typename T> __device__ __forceinline__ float bits_to_f32(uint16_t h);
template <> __device__ __forceinline__ float bits_to_f32<__half>(uint16_t h) { return f16_bits_to_f32(h); }
template <> __device__ __forceinline__ float bits_to_f32<__hip_bfloat16>(uint16_t h) { return bf16_bits_to_f32(h); }

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(__half v) { return __half2float(v); }
__device__ __forceinline__ float to_f32(__hip_bfloat16 v) { return bf16_bits_to_f32(__bfloat16_as_ushort(v)); }

// Exact dequantized values: the fp16 scale widens exactly and the product of
// an 11-bit significand with a code of at most 8 bits is exact in fp32.
__device__ __forceinline__ float q8_value(int8_t q, float d) { return (float)q * d; }
__device__ __forceinline__ float q4_value(int code, float d) { return (float)(code - 8) * d; }

// v & 0x0F0F0F0F: the four low nibbles of v, one per byte.  Written as a
// single v_and_b32 the compiler cannot see through, so that the following
// (float)((r >> 8e) & 0xFF) become one v_cvt_f32_ubyte<e> each instead of a
// v_bfe_u32 + v_cvt_f32_ubyte0 pair.
__device__ __forceinline__ uint32_t nibbles_to_bytes(uint32_t v) {
    uint32_t r;
    asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(v), "v"(0x0F0F0F0Fu));
    return r;
}

// Stores of an fp32 result in the requested output type.
__device__ __forceinline__ void store_out(void* y, int64_t i, float v, int dtype) {
    if (dtype == 0) ((float*)y)[i] = v;                       // MVLM_F32
    else if (dtype == 1) ((uint16_t*)y)[i] = f32_to_f16_bits(v);  // MVLM_F16
    else ((uint16_t*)y)[i] = f32_to_bf16_bits(v);             // MVLM_BF16
}

__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dtype) {
    if (dtype == 0) return ((const float*)p)[i];
    const uint16_t h = ((const uint16_t*)p)[i];
    return dtype == 1 ? f16_bits_to_f32(h) : bf16_bits_to_f32(h);
}

// 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), the tanh form of GELU
// (src/kernels/activations.cl:68)
__device__ __forceinline__ float gelu_tanh(float x) {
    const float u = 0.7978845608f * __builtin_fmaf(0.044715f, x * x * x, x);
    return 0.5f * x * (1.0f + tanhf(u));
}

// x / (1 + exp(-x))  (src/kernels/activations.cl:22)
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// out = act(v + bias[n]) * mul[i] + res[i]  (Epilogue, common.h)
template <class E>
__device__ __forceinline__ float apply_epilogue(const E& e, float v, int64_t i, int64_t n) {
    if (e.bias) v += load_as_f32(e.bias, n, e.dtype);
    if (e.act == 1) v = gelu_tanh(v);
    else if (e.act == 2) v = silu(v);
    if (e.mul) v *= load_as_f32(e.mul, i, e.dtype);
    if (e.res) v += load_as_f32(e.res, i, e.dtype);
    return v;
}

// v + (v of the lane that DPP control `ctrl` names), all lanes valid.
template <int ctrl>
__device__ __forceinline__ float add_dpp(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.  Four
// DPP steps (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror) leave each 16-lane row's sum in all its lanes; the four row
// sums are then read out and added in a fixed order.  No LDS round trips.
__device__ __forceinline__ float wave_sum(float v) {
    v = add_dpp<0xB1>(v);
    v = add_dpp<0x4E>(v);
    v = add_dpp<0x141>(v);
    v = add_dpp<0x140>(v);
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return (r0 + r1) + (r2 + r3);
}

// v of the lane that DPP control `ctrl` names (all lanes valid).
template <int ctrl>
__device__ __forceinline__ float dpp_get(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false));
}

// DPP control that reads, for every lane, a lane of the same 16-lane row whose
// index differs in bit B and agrees in the bits below it: quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_ror:4, row_ror:8.  (The rotations are not pairings,
// but lane i and the lane it reads still differ in bit B only among bits <= B.)
template <int B>
constexpr int kDppFlip = B == 0 ? 0xB1 : B == 1 ? 0x4E : B == 2 ? 0x124 : 0x128;

template <int B, int N>
__device__ __forceinline__ void wave_sum_lanes_step(float (&w)[N], int lane) {
    if constexpr (B < 4) {
        constexpr int cur = (N >> B) > 1 ? (N >> B) : 1;   // values still carried per lane
        if constexpr (cur > 1) {
            // halve: lanes with bit B set keep the odd entries, the others the
            // even ones, and each adds the entry its DPP source does not keep
            const bool up = (lane >> B) & 1;
#pragma unroll
            for (int k = 0; k < cur / 2; ++k) {
                const float keep = up ? w[2 * k + 1] : w[2 * k];
                const float give = up ? w[2 * k] : w[2 * k + 1];
                w[k] = keep + dpp_get<kDppFlip<B>>(give);
            }
        } else {
            w[0] += dpp_get<kDppFlip<B>>(w[0]);
        }
        wave_sum_lanes_step<B + 1, N>(w, lane);
    }
}

// Sums each of v[0..N) over the 64 lanes of a wavefront (N = 1, 2, 4, 8, 16);
// lane l receives the total of index l & (N - 1).  The values are halved
// across lanes first (one DPP add per pair and step), so N sums cost about
// 3N + 6 instructions instead of N full reductions, and the N totals end up
// in N different lanes.  Row sums are combined with two lane shuffles.
template <int N>
__device__ __forceinline__ float wave_sum_lanes(const float (&v)[N], int lane) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "power of two up to 16");
    float w[N];
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = v[i];
    wave_sum_lanes_step<0, N>(w, lane);
    float t = w[0];
    t += __shfl_xor(t, 16);
    t += __shfl_xor(t, 32);
    return t;
}

// LDS pointer type of the direct global->LDS loads (global_load_lds_*): lane i
// of the instruction writes its bytes at base + i * width.
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt with vmcnt = n, expcnt and lgkmcnt unconstrained (gfx9 encoding).
// Direct LDS loads count in vmcnt like other vector loads, in issue order.
// (The compiler may strengthen this wait but keeps it; it also adds its own
// waits for LDS reads it can see.)
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ---- LDS reads the compiler does not track ------------------------------------
// The compiler inserts a full vmcnt(0) before any LDS read that may alias an
// in-flight direct global->LDS load, and merges loop-carried LDS reads into
// lgkmcnt(0), both of which serialize a software pipeline.  Kernels that
// manage their own waits read LDS with these inline-asm loads instead, and
// must then order everything by hand:
//  * asm_wait_vmcnt<n>() before reading LDS filled by direct loads (and a
//    barrier when other waves filled it);
//  * asm_wait_lgkmcnt<n>() and then asm_pin(reg) on each loaded register
//    before using it, so no use can be scheduled above the wait.  LDS reads
//    complete in issue order.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
template <int OFF = 0>
__device__ __forceinline__ u32x4 asm_lds_read_b128(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
template <int OFF = 0>
__device__ __forceinline__ u32x2 asm_lds_read_b64(uint32_t addr) {
    u32x2 v;
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
template <int OFF = 0>
__device__ __forceinline__ uint32_t asm_lds_read_u16(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF) : "memory");
    return v;
}
// A direct global->LDS 16-byte load the compiler does not track: lane i's 16
// bytes from gaddr land at LDS byte lds_base + 16 * i (lds_base wave-uniform).
// The compiler puts a vmcnt(0) in front of every tracked direct load that may
// overwrite LDS written by an earlier one, which caps a multi-stage ring at
// one stage in flight; with this form the kernel's own waits order the ring.
// M0 is reserved to the compiler, which sets it before each of its own uses
// (direct loads, GWS, messages; LDS reads/writes do not use it on gfx950), so
// the clobber below documents the write rather than being needed.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void asm_global_load_lds_b128(const void* gaddr, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(gaddr), "s"(lds_base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// The buffer-addressed form of the same direct load: lane i's 16 bytes at
// byte voff of the buffer described by rsrc (four wave-uniform words: base,
// base high | stride 0, size in bytes, format) land at LDS byte
// lds_base + 16 * i.  A 32-bit offset per lane instead of a 64-bit address.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 raw_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return i32x4{(int)__builtin_amdgcn_readfirstlane((uint32_t)a),
                 (int)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xFFFFu),
                 (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000};
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void asm_buffer_load_lds_b128(i32x4 rsrc, uint32_t voff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :
                 : "v"(voff), "s"(rsrc), "s"(lds_base)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// A 16-byte buffer load the compiler does not track (wait with
// asm_wait_vmcnt, then asm_pin the result).
__device__ __forceinline__ u32x4 asm_buffer_load_b128(i32x4 rsrc, uint32_t voff) {
    u32x4 v;
    asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rsrc) : "memory");
    return v;
}
// A 16-byte global load the compiler does not track (wait with
// asm_wait_vmcnt, then asm_pin the result).
__device__ __forceinline__ u32x4 asm_global_load_b128(const void* p) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
    return v;
}
// Global stores that write through the XCD's L2 (sc1), for kernels whose
// output runs to tens of MB: the data leaves for HBM as it is written instead
// of sitting in L2 as dirty lines that the end of the kernel has to write
// back (prefill GEMMs 8-10% faster).  The compiler does not count these in
// vmcnt; a wait it computes for an earlier load is then only stricter.
__device__ __forceinline__ void asm_global_store_b128_wt(void* p, u32x4 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void asm_global_store_b64_wt(void* p, u32x2 v) {
    asm volatile("global_store_dwordx2 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
template <int n>
__device__ __forceinline__ void asm_wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}
template <int n>
__device__ __forceinline__ void asm_wait_lgkmcnt() {
    static_assert(n >= 0 && n < 16, "lgkmcnt range");
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(n) : "memory");
}
// Ties a register to the preceding wait: an empty volatile asm that "writes"
// r, so every use of r is scheduled after the wait.
template <typename T>
__device__ __forceinline__ void asm_pin(T& r) {
    asm volatile("" : "+v"(r));
}

}  // namespace mvlm
