// mgpu_engine.cpp — the reference's engine API (device/memory/compute, GEMM
// and GEMV part) implemented over the C ABI.  See mgpu_engine.h.
#include "mgpu_engine.h"

#include <cstdio>

namespace mgpu {

namespace {

// Logs the failing call like CL_CHECK_NULL (src/engine/compute.cpp:12-17).
bool ok(int status, const char* what) {
    if (status == MVLM_OK) return true;
    std::fprintf(stderr, "MGPU error %d in %s: %s\n", status, what, mvlm_last_error());
    return false;
}

}  // namespace

bool init_device(DeviceInfo* info) {
    if (!info) return false;
    mvlm_device* dev = nullptr;
    if (!ok(mvlm_device_create(0, &dev), "init_device")) return false;
    mvlm_device_info di{};
    if (!ok(mvlm_device_get_info(dev, &di), "init_device")) {
        mvlm_device_destroy(dev);
        return false;
    }
    info->device = dev;
    std::snprintf(info->device_name, sizeof(info->device_name), "%s", di.device_name);
    std::snprintf(info->arch_name, sizeof(info->arch_name), "%s", di.arch_name);
    info->compute_units = (unsigned)di.compute_units;
    info->max_clock_freq = (unsigned)di.max_clock_mhz;
    info->global_mem_size = di.global_mem_size;
    info->local_mem_size = di.local_mem_size;
    info->has_fp16 = true;
    return true;
}

void print_device_info(const DeviceInfo* info) {
    if (!info) return;
    std::printf("Device: %s (%s)\n  Compute units: %u\n  Max clock: %u MHz\n  Global memory: %.1f GiB\n"
                "  LDS per work-group: %llu KiB\n",
                info->device_name, info->arch_name, info->compute_units, info->max_clock_freq,
                (double)info->global_mem_size / (1024.0 * 1024.0 * 1024.0),
                (unsigned long long)(info->local_mem_size / 1024));
}

void destroy_device(DeviceInfo* info) {
    if (!info || !info->device) return;
    ok(mvlm_device_destroy(info->device), "destroy_device");
    info->device = nullptr;
}

bool finish(const DeviceInfo* info) {
    return info && ok(mvlm_device_synchronize(info->device), "finish");
}

Weight create_weight_image(const DeviceInfo* info, int rows, int cols, const half_bits* data) {
    if (!info) return nullptr;
    mvlm_weight* w = nullptr;
    // rows = K, cols = N: the [K][N] layout the reference's kernels index
    return ok(mvlm_weight_pack(info->device, data, MVLM_F16, MVLM_LAYOUT_KN, cols, rows, &w), "create_weight_image")
               ? w : nullptr;
}

Weight create_weight(const DeviceInfo* info, int ggml_type, int N, int K, const void* data) {
    if (!info) return nullptr;
    mvlm_weight* w = nullptr;
    return ok(mvlm_weight_pack(info->device, data, ggml_type, MVLM_LAYOUT_NK, N, K, &w), "create_weight") ? w : nullptr;
}

Buffer create_buffer(const DeviceInfo* info, size_t size_bytes, int /*flags*/, void* host_ptr) {
    if (!info) return nullptr;
    mvlm_buffer* b = nullptr;
    if (!ok(mvlm_buffer_alloc(info->device, size_bytes, &b), "create_buffer")) return nullptr;
    if (host_ptr && !ok(mvlm_buffer_upload(b, 0, host_ptr, size_bytes), "create_buffer")) {
        mvlm_buffer_free(b);
        return nullptr;
    }
    return b;
}

void release_buffer(Buffer buf) {
    if (buf) ok(mvlm_buffer_free(buf), "release_buffer");
}

void release_weight(Weight w) {
    if (w) ok(mvlm_weight_free(w), "release_weight");
}

bool read_buffer(const DeviceInfo* info, Buffer buf, size_t offset, size_t bytes, void* dst) {
    return info && ok(mvlm_buffer_download(buf, offset, dst, bytes), "read_buffer");
}

bool init_buffer_pool(BufferPool* pool, const DeviceInfo* info, size_t size_bytes) {
    if (!pool || !info) return false;
    pool->buffers[0] = pool->buffers[1] = nullptr;
    pool->size = size_bytes;
    pool->current = 0;
    pool->buffers[0] = create_buffer(info, size_bytes);
    if (!pool->buffers[0]) return false;
    pool->buffers[1] = create_buffer(info, size_bytes);
    if (!pool->buffers[1]) {
        release_buffer(pool->buffers[0]);
        pool->buffers[0] = nullptr;
        return false;
    }
    return true;
}

Buffer get_current_buffer(BufferPool* pool) { return pool->buffers[pool->current]; }
Buffer get_next_buffer(BufferPool* pool) { return pool->buffers[1 - pool->current]; }
void swap_buffers(BufferPool* pool) { pool->current = 1 - pool->current; }

void destroy_buffer_pool(BufferPool* pool) {
    for (int i = 0; i < 2; ++i) {
        release_buffer(pool->buffers[i]);
        pool->buffers[i] = nullptr;
    }
    pool->size = 0;
    pool->current = 0;
}

Event dispatch_gemm_naive(const DeviceInfo* dev, Program, Buffer A, Buffer B, Buffer C, int M, int N, int K) {
    mvlm_event* ev = nullptr;
    return dev && ok(mvlm_gemm_naive(dev->device, A, B, C, M, N, K, &ev), "dispatch_gemm_naive") ? ev : nullptr;
}

Event dispatch_gemm_tiled(const DeviceInfo* dev, Program, Buffer A, Buffer B, Buffer C, int M, int N, int K) {
    mvlm_event* ev = nullptr;
    return dev && ok(mvlm_gemm_tiled(dev->device, A, B, C, M, N, K, &ev), "dispatch_gemm_tiled") ? ev : nullptr;
}

Event dispatch_gemm_image(const DeviceInfo* dev, Program, Buffer A, Weight B_img, Buffer C, int M, int N, int K) {
    mvlm_event* ev = nullptr;
    return dev && ok(mvlm_gemm_packed(dev->device, A, MVLM_F16, B_img, C, MVLM_F16, M, N, K, &ev),
                     "dispatch_gemm_image") ? ev : nullptr;
}

Event dispatch_gemv(const DeviceInfo* dev, Program, Buffer x, Weight W_img, Buffer y, int N, int K) {
    mvlm_event* ev = nullptr;
    return dev && ok(mvlm_gemv(dev->device, x, MVLM_F16, W_img, y, MVLM_F16, N, K, &ev), "dispatch_gemv") ? ev
                                                                                                    : nullptr;
}

Event dispatch_gemv_exact(const DeviceInfo* dev, Program, Buffer x, Weight W_img, Buffer y, int N, int K) {
    mvlm_event* ev = nullptr;
    return dev && ok(mvlm_gemv_exact(dev->device, x, W_img, y, N, K, &ev), "dispatch_gemv_exact") ? ev : nullptr;
}

Event dispatch_gemv_quant(const DeviceInfo* dev, Program, Buffer x, Weight W, Buffer y, int M, int N, int K) {
    if (!dev || !W) return nullptr;
    mvlm_event* ev = nullptr;
    int st = mvlm_weight_dtype(W) == MVLM_Q4_0 ? mvlm_gemm_q4_0(dev->device, x, W, y, M, N, K, &ev)
                                               : mvlm_gemm_q8_0(dev->device, x, W, y, M, N, K, &ev);
    return ok(st, "dispatch_gemv_quant") ? ev : nullptr;
}

Event dispatch_attention_prefill(const DeviceInfo* dev, Program, Buffer Q, Buffer K, Buffer V, Buffer output,
                                 int seq_len, int num_heads, int head_dim) {
    if (!dev) return nullptr;
    mvlm_event* ev = nullptr;
    int st = mvlm_attention_prefill(dev->device, Q, K, V, output, seq_len, num_heads, head_dim, &ev);
    return ok(st, "dispatch_attention_prefill") ? ev : nullptr;
}

Event dispatch_attention_decode(const DeviceInfo* dev, Program, Buffer Q, Buffer K_cache, Buffer V_cache,
                                Buffer output, int cache_len, int num_heads, int head_dim) {
    if (!dev) return nullptr;
    mvlm_event* ev = nullptr;
    int st = mvlm_attention_decode(dev->device, Q, K_cache, V_cache, output, cache_len, num_heads, head_dim, &ev);
    return ok(st, "dispatch_attention_decode") ? ev : nullptr;
}

int argmax_logits(const DeviceInfo* dev, Buffer logits, int vocab_size) {
    if (!dev) return -1;
    mvlm_buffer* out = nullptr;
    if (!ok(mvlm_buffer_alloc(dev->device, 4, &out), "argmax_logits")) return -1;
    int32_t id = -1;
    bool good = ok(mvlm_argmax(dev->device, logits, MVLM_F16, 1, vocab_size, vocab_size, out, nullptr), "argmax_logits") &&
                ok(mvlm_buffer_download(out, 0, &id, 4), "argmax_logits");
    mvlm_buffer_free(out);
    return good ? id : -1;
}

bool wait_event(Event ev) { return ev && ok(mvlm_event_wait(ev), "wait_event"); }

double event_elapsed_ms(Event ev) {
    float ms = 0.0f;
    return (ev && ok(mvlm_event_elapsed_ms(ev, &ms), "event_elapsed_ms")) ? (double)ms : -1.0;
}

void release_event(Event ev) {
    if (ev) ok(mvlm_event_release(ev), "release_event");
}

}  // namespace mgpu
