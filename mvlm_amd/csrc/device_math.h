// Device-side number-format helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <cstdint>

namespace mvlm {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
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

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace mvlm
