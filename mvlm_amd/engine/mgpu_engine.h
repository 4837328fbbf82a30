// mgpu_engine.h — C++ drop-in for the matmul part of MVLM's engine API.
//
// Mirrors, over the C ABI of include/mvlm_hip.h:
//   src/engine/device.h:13-75    DeviceInfo, init_device, destroy_device, print_device_info
//   src/engine/memory.h:15-35    create_weight_image, create_buffer, BufferPool + helpers
//   src/engine/compute.h:13-33   dispatch_gemm_naive / _tiled / _image, dispatch_gemv
// with the same names, argument order and meaning.  OpenCL handles become
// opaque HIP-side handles: cl_mem -> Buffer (activations) or Weight (packed
// weights from create_weight_image), cl_event -> Event.  The cl_program
// argument is kept so call sites change only in types; the gfx950 kernels are
// part of the library, so it is ignored.  Errors keep the reference's
// behaviour: the message goes to stderr and the function returns nullptr
// (or false), as CL_CHECK_NULL does (src/engine/compute.cpp:12-17).
#pragma once

#include <cstddef>
#include <cstdint>

#include "mvlm_hip.h"

namespace mgpu {

using Buffer = mvlm_buffer*;
using Weight = mvlm_weight*;
using Event = mvlm_event*;
using Program = const void*;     // stands in for cl_program; ignored
using half_bits = uint16_t;      // cl_half

struct DeviceInfo {
    mvlm_device* device = nullptr;
    char device_name[256] = {};
    char arch_name[64] = {};
    unsigned compute_units = 0;
    unsigned max_clock_freq = 0;     // MHz
    uint64_t global_mem_size = 0;
    uint64_t local_mem_size = 0;
    bool has_fp16 = true;
};

// ---- device (src/engine/device.h:58-75) ----
bool init_device(DeviceInfo* info);
void print_device_info(const DeviceInfo* info);
void destroy_device(DeviceInfo* info);
bool finish(const DeviceInfo* info);                  // clFinish

// ---- memory (src/engine/memory.h:15-35) ----
// rows x cols fp16, row-major, as the reference passes it (rows = K, cols = N).
Weight create_weight_image(const DeviceInfo* info, int rows, int cols, const half_bits* data);
// GGUF-native [N][K] weight of any supported type (F32/F16/BF16/Q8_0/Q4_0).
Weight create_weight(const DeviceInfo* info, int ggml_type, int N, int K, const void* data);
// flags are accepted for source compatibility; host_ptr != nullptr copies its
// contents in (CL_MEM_COPY_HOST_PTR).
Buffer create_buffer(const DeviceInfo* info, size_t size_bytes, int flags = 0, void* host_ptr = nullptr);
void release_buffer(Buffer buf);
void release_weight(Weight w);
bool read_buffer(const DeviceInfo* info, Buffer buf, size_t offset, size_t bytes, void* dst);

struct BufferPool {
    Buffer buffers[2] = {nullptr, nullptr};
    size_t size = 0;
    int current = 0;
};
bool init_buffer_pool(BufferPool* pool, const DeviceInfo* info, size_t size_bytes);
Buffer get_current_buffer(BufferPool* pool);
Buffer get_next_buffer(BufferPool* pool);
void swap_buffers(BufferPool* pool);
void destroy_buffer_pool(BufferPool* pool);

// ---- compute (src/engine/compute.h:13-33) ----
// C[M,N] = A[M,K] * B[K,N], fp16 in / fp16 out, fp32 fma in ascending k.
Event dispatch_gemm_naive(const DeviceInfo* dev, Program program, Buffer A, Buffer B, Buffer C, int M, int N, int K);
Event dispatch_gemm_tiled(const DeviceInfo* dev, Program program, Buffer A, Buffer B, Buffer C, int M, int N, int K);
// C[M,N] = A[M,K] * B_img, B_img from create_weight_image; fp16 out, MFMA.
Event dispatch_gemm_image(const DeviceInfo* dev, Program program, Buffer A, Weight B_img, Buffer C, int M, int N, int K);
// y[1,N] = x[1,K] * W_img; fp16 x and y.
Event dispatch_gemv(const DeviceInfo* dev, Program program, Buffer x, Weight W_img, Buffer y, int N, int K);
// Same product with gemv's summation order (gemm.cl:215-270): bit-identical y.
Event dispatch_gemv_exact(const DeviceInfo* dev, Program program, Buffer x, Weight W_img, Buffer y, int N, int K);
// The dequantizing GEMV of README.md:57 (fp32 x and y, Q8_0 / Q4_0 weights), M <= 16 rows.
Event dispatch_gemv_quant(const DeviceInfo* dev, Program program, Buffer x, Weight W, Buffer y, int M, int N, int K);
// src/engine/compute.h:65-73 (fused MFMA attention; fp16 [seq][heads][head_dim])
Event dispatch_attention_prefill(const DeviceInfo* dev, Program program, Buffer Q, Buffer K, Buffer V, Buffer output,
                                 int seq_len, int num_heads, int head_dim);
Event dispatch_attention_decode(const DeviceInfo* dev, Program program, Buffer Q, Buffer K_cache, Buffer V_cache,
                                Buffer output, int cache_len, int num_heads, int head_dim);
// replaces argmax_logits (src/models/moondream2.cpp:553-593): the token id of
// the largest fp16 logit, picked on the device (4 bytes read back); -1 on error
int argmax_logits(const DeviceInfo* dev, Buffer logits, int vocab_size);

// cl_event handling: clWaitForEvents + profiling read + clReleaseEvent.
bool wait_event(Event ev);
double event_elapsed_ms(Event ev);
void release_event(Event ev);

}  // namespace mgpu
