// Host runtime of the C ABI: device, buffers, pool, packed weights, events,
// and the validated launch entry points.  Argument checks happen here, on the
// host, before anything is enqueued; kernels assume validated shapes.
#include "common.h"

#include <cstdlib>
#include <cstring>
#include <new>

namespace mvlm {

static thread_local std::string g_last_error;

KernelTiming& kernel_timing() {
    static thread_local KernelTiming t;
    return t;
}

static bool quiet() {
    static const bool q = [] {   // read once, thread-safe initialisation
        const char* e = std::getenv("MVLM_QUIET");
        return e && *e && *e != '0';
    }();
    return q;
}

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    if (!quiet()) fprintf(stderr, "mvlm: %s\n", buf);
    return code;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return MVLM_OK;
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
        return set_error(MVLM_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
    return set_error(MVLM_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

LaunchScope::LaunchScope(mvlm_device* d, mvlm_event** o) : dev(d), out(o) {
    if (out) {
        *out = nullptr;
        ev = new (std::nothrow) mvlm_event();
        if (!ev) { status = set_error(MVLM_ERR_OUT_OF_MEMORY, "event allocation failed"); return; }
        ev->dev = dev;
        status = check_hip(hipEventCreate(&ev->start), "hipEventCreate");
        if (status == MVLM_OK) status = check_hip(hipEventCreate(&ev->end), "hipEventCreate");
        if (status == MVLM_OK) status = check_hip(hipEventRecord(ev->start, dev->stream), "hipEventRecord");
    }
}

int LaunchScope::finish(const char* kernel_name) {
    hipError_t le = hipGetLastError();
    if (le != hipSuccess) status = check_hip(le, kernel_name);
    if (ev) {
        if (status == MVLM_OK) status = check_hip(hipEventRecord(ev->end, dev->stream), "hipEventRecord");
        if (status == MVLM_OK) {
            *out = ev;
        } else {
            if (ev->start) (void)hipEventDestroy(ev->start);
            if (ev->end) (void)hipEventDestroy(ev->end);
            delete ev;
        }
        ev = nullptr;
    }
    return status;
}

}  // namespace mvlm

using namespace mvlm;


// ---------------------------------------------------------------------------
// errors / version
// ---------------------------------------------------------------------------

extern "C" const char* mvlm_last_error(void) { return g_last_error.c_str(); }
extern "C" int mvlm_abi_version(void) { return MVLM_ABI_VERSION; }

// ---------------------------------------------------------------------------
// device
// ---------------------------------------------------------------------------

extern "C" int mvlm_device_count(int* count) {
    REQUIRE(count, "mvlm_device_count: count is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;   // no driver / no device: zero devices, not an error
    *count = n;
    (void)hipGetLastError();
    return MVLM_OK;
}

extern "C" int mvlm_device_create(int ordinal, mvlm_device** out) {
    REQUIRE(out, "mvlm_device_create: out is null");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return set_error(MVLM_ERR_NO_DEVICE, "no HIP device available");
    }
    if (ordinal < 0 || ordinal >= n)
        return set_error(MVLM_ERR_NO_DEVICE, "device ordinal %d out of range (%d devices)", ordinal, n);
    HIP_TRY(hipSetDevice(ordinal));
    mvlm_device* d = new (std::nothrow) mvlm_device();
    if (!d) return set_error(MVLM_ERR_OUT_OF_MEMORY, "device allocation failed");
    d->ordinal = ordinal;
    int st = check_hip(hipGetDeviceProperties(&d->prop, ordinal), "hipGetDeviceProperties");
    if (st == MVLM_OK) st = check_hip(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking), "hipStreamCreate");
    if (st == MVLM_OK) st = resolve_noalloc_scratch(d);
    if (st != MVLM_OK) {
        if (d->stream) (void)hipStreamDestroy(d->stream);
        delete d;
        return st;
    }
    *out = d;
    return MVLM_OK;
}

extern "C" int mvlm_device_destroy(mvlm_device* dev) {
    REQUIRE(dev, "mvlm_device_destroy: dev is null");
    (void)hipSetDevice(dev->ordinal);
    int st = MVLM_OK;
    if (dev->stream) {
        st = check_hip(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
        int st2 = check_hip(hipStreamDestroy(dev->stream), "hipStreamDestroy");
        if (st == MVLM_OK) st = st2;
    }
    for (void* p : dev->scratch_blocks) (void)hipFree(p);
    if (dev->sync_words) (void)hipFree(dev->sync_words);
    delete dev;
    return st;
}

namespace mvlm {
int device_scratch(mvlm_device* dev, size_t bytes, void** out) {
    *out = nullptr;
    if (bytes == 0) return MVLM_OK;
    if (bytes > dev->scratch_bytes) {
        HIP_TRY(hipSetDevice(dev->ordinal));
        const size_t want = (bytes + 0xFFFFF) & ~(size_t)0xFFFFF;      // whole MiB
        void* p = nullptr;
        if (hipMalloc(&p, want) != hipSuccess || !p) {
            (void)hipGetLastError();
            return set_error(MVLM_ERR_OUT_OF_MEMORY, "workspace allocation of %zu bytes failed", want);
        }
        try {
            dev->scratch_blocks.push_back(p);
        } catch (...) {
            (void)hipFree(p);
            return set_error(MVLM_ERR_OUT_OF_MEMORY, "workspace bookkeeping failed");
        }
        dev->scratch_bytes = want;
    }
    *out = dev->scratch_blocks.back();
    return MVLM_OK;
}

int device_sync_words(mvlm_device* dev, void** out) {
    if (!dev->sync_words) {
        HIP_TRY(hipSetDevice(dev->ordinal));
        void* p = nullptr;
        if (hipMalloc(&p, SYNC_WORDS_BYTES) != hipSuccess || !p) {
            (void)hipGetLastError();
            return set_error(MVLM_ERR_OUT_OF_MEMORY, "sync word allocation failed");
        }
        if (hipMemsetAsync(p, 0, SYNC_WORDS_BYTES, dev->stream) != hipSuccess ||
            hipStreamSynchronize(dev->stream) != hipSuccess) {
            (void)hipFree(p);
            return set_error(MVLM_ERR_HIP, "sync word initialisation failed");
        }
        dev->sync_words = p;
    }
    *out = dev->sync_words;
    return MVLM_OK;
}
}  // namespace mvlm

extern "C" int mvlm_device_get_info(const mvlm_device* dev, mvlm_device_info* info) {
    REQUIRE(dev && info, "mvlm_device_get_info: null argument");
    std::memset(info, 0, sizeof(*info));
    const hipDeviceProp_t& p = dev->prop;
    std::snprintf(info->device_name, sizeof(info->device_name), "%s", p.name);
    std::snprintf(info->arch_name, sizeof(info->arch_name), "%s", p.gcnArchName);
    info->ordinal = dev->ordinal;
    info->compute_units = p.multiProcessorCount;
    info->max_clock_mhz = p.clockRate / 1000;
    info->memory_clock_mhz = p.memoryClockRate / 1000;
    info->memory_bus_width_bits = p.memoryBusWidth;
    info->wavefront_size = p.warpSize;
    info->global_mem_size = p.totalGlobalMem;
    info->local_mem_size = p.sharedMemPerBlock;
    info->l2_cache_size = (uint64_t)p.l2CacheSize;
    info->peak_hbm_gbs = 8000.0;
    info->peak_fp16_tflops = 2500.0;
    info->box_peak_hbm_gbs = (double)info->memory_clock_mhz * 1e6 * info->memory_bus_width_bits * 4.0 / 8.0 / 1e9;
    info->box_peak_fp16_tflops = (double)info->compute_units * info->max_clock_mhz * 1e6 * 4096.0 / 1e12;
    return MVLM_OK;
}

extern "C" int mvlm_device_synchronize(mvlm_device* dev) {
    REQUIRE(dev, "mvlm_device_synchronize: dev is null");
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return MVLM_OK;
}

// ---------------------------------------------------------------------------
// buffers
// ---------------------------------------------------------------------------

extern "C" int mvlm_buffer_alloc(mvlm_device* dev, size_t bytes, mvlm_buffer** out) {
    REQUIRE(dev && out, "mvlm_buffer_alloc: null argument");
    *out = nullptr;
    REQUIRE(bytes > 0, "mvlm_buffer_alloc: size must be positive");
    HIP_TRY(hipSetDevice(dev->ordinal));
    void* p = nullptr;
    HIP_TRY(hipMalloc(&p, bytes));
    mvlm_buffer* b = new (std::nothrow) mvlm_buffer();
    if (!b) { (void)hipFree(p); return set_error(MVLM_ERR_OUT_OF_MEMORY, "buffer allocation failed"); }
    b->dev = dev; b->ptr = p; b->bytes = bytes; b->owned = true;
    *out = b;
    return MVLM_OK;
}

extern "C" int mvlm_buffer_view(mvlm_buffer* parent, size_t offset, size_t bytes, mvlm_buffer** out) {
    REQUIRE(parent && out, "mvlm_buffer_view: null argument");
    *out = nullptr;
    REQUIRE(bytes > 0 && offset <= parent->bytes && bytes <= parent->bytes - offset,
            "mvlm_buffer_view: [%zu, %zu) outside a buffer of %zu bytes", offset, offset + bytes, parent->bytes);
    mvlm_buffer* b = new (std::nothrow) mvlm_buffer();
    if (!b) return set_error(MVLM_ERR_OUT_OF_MEMORY, "buffer allocation failed");
    b->dev = parent->dev; b->ptr = (char*)parent->ptr + offset; b->bytes = bytes;
    b->owned = false; b->parent = parent;
    parent->views++;
    *out = b;
    return MVLM_OK;
}

extern "C" int mvlm_buffer_free(mvlm_buffer* buf) {
    REQUIRE(buf, "mvlm_buffer_free: buf is null");
    REQUIRE(buf->views == 0, "mvlm_buffer_free: %d views of this buffer are still alive", buf->views);
    int st = MVLM_OK;
    if (buf->owned) {
        (void)hipSetDevice(buf->dev->ordinal);
        st = check_hip(hipFree(buf->ptr), "hipFree");
    } else if (buf->parent) {
        buf->parent->views--;
    }
    delete buf;
    return st;
}

extern "C" size_t mvlm_buffer_size(const mvlm_buffer* buf) { return buf ? buf->bytes : 0; }

extern "C" int mvlm_buffer_upload(mvlm_buffer* buf, size_t offset, const void* src, size_t bytes) {
    REQUIRE(buf && (src || bytes == 0), "mvlm_buffer_upload: null argument");
    REQUIRE(offset <= buf->bytes && bytes <= buf->bytes - offset,
            "mvlm_buffer_upload: %zu bytes at offset %zu exceed a buffer of %zu bytes", bytes, offset, buf->bytes);
    if (bytes == 0) return MVLM_OK;
    HIP_TRY(hipMemcpyAsync((char*)buf->ptr + offset, src, bytes, hipMemcpyHostToDevice, buf->dev->stream));
    HIP_TRY(hipStreamSynchronize(buf->dev->stream));
    return MVLM_OK;
}

extern "C" int mvlm_buffer_download(const mvlm_buffer* buf, size_t offset, void* dst, size_t bytes) {
    REQUIRE(buf && (dst || bytes == 0), "mvlm_buffer_download: null argument");
    REQUIRE(offset <= buf->bytes && bytes <= buf->bytes - offset,
            "mvlm_buffer_download: %zu bytes at offset %zu exceed a buffer of %zu bytes", bytes, offset, buf->bytes);
    if (bytes == 0) return MVLM_OK;
    HIP_TRY(hipMemcpyAsync(dst, (const char*)buf->ptr + offset, bytes, hipMemcpyDeviceToHost, buf->dev->stream));
    HIP_TRY(hipStreamSynchronize(buf->dev->stream));
    return MVLM_OK;
}

extern "C" int mvlm_buffer_fill_zero(mvlm_buffer* buf) {
    REQUIRE(buf, "mvlm_buffer_fill_zero: buf is null");
    HIP_TRY(hipMemsetAsync(buf->ptr, 0, buf->bytes, buf->dev->stream));
    return MVLM_OK;
}

// ---------------------------------------------------------------------------
// ping-pong pool
// ---------------------------------------------------------------------------

extern "C" int mvlm_pool_init(mvlm_device* dev, size_t bytes, mvlm_pool** out) {
    REQUIRE(dev && out, "mvlm_pool_init: null argument");
    *out = nullptr;
    mvlm_pool* p = new (std::nothrow) mvlm_pool();
    if (!p) return set_error(MVLM_ERR_OUT_OF_MEMORY, "pool allocation failed");
    int st = mvlm_buffer_alloc(dev, bytes, &p->buffers[0]);
    if (st == MVLM_OK) {
        st = mvlm_buffer_alloc(dev, bytes, &p->buffers[1]);
        if (st != MVLM_OK) { mvlm_buffer_free(p->buffers[0]); p->buffers[0] = nullptr; }
    }
    if (st != MVLM_OK) { delete p; return st; }
    p->size = bytes;
    p->current = 0;
    *out = p;
    return MVLM_OK;
}

extern "C" mvlm_buffer* mvlm_pool_current(mvlm_pool* pool) { return pool ? pool->buffers[pool->current] : nullptr; }
extern "C" mvlm_buffer* mvlm_pool_next(mvlm_pool* pool) { return pool ? pool->buffers[1 - pool->current] : nullptr; }

extern "C" int mvlm_pool_swap(mvlm_pool* pool) {
    REQUIRE(pool, "mvlm_pool_swap: pool is null");
    pool->current = 1 - pool->current;
    return MVLM_OK;
}

extern "C" int mvlm_pool_destroy(mvlm_pool* pool) {
    REQUIRE(pool, "mvlm_pool_destroy: pool is null");
    int st = MVLM_OK;
    for (int i = 0; i < 2; ++i)
        if (pool->buffers[i]) {
            int s = mvlm_buffer_free(pool->buffers[i]);
            if (st == MVLM_OK) st = s;
        }
    delete pool;
    return st;
}

// ---------------------------------------------------------------------------
// packed weights
// ---------------------------------------------------------------------------

static int weight_alloc(mvlm_device* dev, int dtype, int N, int K, mvlm_weight** out) {
    *out = nullptr;
    REQUIRE(is_dense(dtype) || is_quant(dtype), "weight: unsupported dtype %d", dtype);
    REQUIRE(N > 0 && K > 0, "weight: N=%d and K=%d must be positive", N, K);
    if (is_quant(dtype)) REQUIRE(K % 32 == 0, "weight: quantized K=%d is not a multiple of 32", K);
    mvlm_weight* w = new (std::nothrow) mvlm_weight();
    if (!w) return set_error(MVLM_ERR_OUT_OF_MEMORY, "weight allocation failed");
    w->dev = dev; w->dtype = dtype; w->N = N; w->K = K;
    size_t data_bytes, scale_bytes = 0;
    if (is_dense(dtype)) {
        w->ld = round_up(K, 64);
        data_bytes = (size_t)N * (size_t)w->ld * dtype_size(dtype);
    } else {
        w->ld = (dtype == MVLM_Q8_0) ? K : K / 2;
        data_bytes = (size_t)N * (size_t)w->ld;
        scale_bytes = (size_t)N * (size_t)(K / 32) * 2;
    }
    size_t data_pad = (size_t)round_up((int64_t)data_bytes, 256);
    w->bytes = data_bytes + scale_bytes;
    (void)hipSetDevice(dev->ordinal);
    int st = check_hip(hipMalloc(&w->alloc, data_pad + scale_bytes + 256), "hipMalloc(weight)");
    if (st != MVLM_OK) { delete w; return st; }
    w->data = w->alloc;
    w->scales = scale_bytes ? (char*)w->alloc + data_pad : nullptr;
    *out = w;
    return MVLM_OK;
}

static size_t source_bytes(int dtype, int N, int K) {
    if (dtype == MVLM_Q8_0) return (size_t)N * (K / 32) * 34;
    if (dtype == MVLM_Q4_0) return (size_t)N * (K / 32) * 18;
    return (size_t)N * (size_t)K * dtype_size(dtype);
}

static int check_pack_args(mvlm_device* dev, int dtype, int layout, int N, int K, mvlm_weight** out) {
    REQUIRE(dev && out, "mvlm_weight_pack: null argument");
    *out = nullptr;
    REQUIRE(is_dense(dtype) || is_quant(dtype), "mvlm_weight_pack: unsupported dtype %d", dtype);
    REQUIRE(layout == MVLM_LAYOUT_NK || layout == MVLM_LAYOUT_KN, "mvlm_weight_pack: bad layout %d", layout);
    REQUIRE(N > 0 && K > 0, "mvlm_weight_pack: N=%d and K=%d must be positive", N, K);
    if (is_quant(dtype)) {
        REQUIRE(layout == MVLM_LAYOUT_NK, "mvlm_weight_pack: quantized weights must be GGUF blocks along K (layout NK)");
        REQUIRE(K % 32 == 0, "mvlm_weight_pack: quantized K=%d is not a multiple of 32", K);
    }
    return MVLM_OK;
}

extern "C" int mvlm_weight_pack_device(mvlm_device* dev, const mvlm_buffer* src, int dtype, int layout,
                                       int N, int K, mvlm_weight** out) {
    int st = check_pack_args(dev, dtype, layout, N, K, out);
    if (st != MVLM_OK) return st;
    REQUIRE(src, "mvlm_weight_pack_device: src is null");
    size_t need = source_bytes(dtype, N, K);
    if (src->bytes < need)
        return set_error(MVLM_ERR_BUFFER_TOO_SMALL, "mvlm_weight_pack_device: source holds %zu bytes, %zu needed",
                         src->bytes, need);
    mvlm_weight* w = nullptr;
    st = weight_alloc(dev, dtype, N, K, &w);
    if (st != MVLM_OK) return st;
    st = check_hip(launch_pack(dev->stream, src->ptr, dtype, layout, N, K, w), "pack kernel");
    if (st == MVLM_OK) st = check_hip(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
    if (st != MVLM_OK) { (void)hipFree(w->alloc); delete w; return st; }
    *out = w;
    return MVLM_OK;
}

extern "C" int mvlm_weight_pack(mvlm_device* dev, const void* src, int dtype, int layout,
                                int N, int K, mvlm_weight** out) {
    int st = check_pack_args(dev, dtype, layout, N, K, out);
    if (st != MVLM_OK) return st;
    REQUIRE(src, "mvlm_weight_pack: src is null");
    mvlm_buffer* staging = nullptr;
    size_t bytes = source_bytes(dtype, N, K);
    st = mvlm_buffer_alloc(dev, bytes, &staging);
    if (st != MVLM_OK) return st;
    st = mvlm_buffer_upload(staging, 0, src, bytes);
    if (st == MVLM_OK) st = mvlm_weight_pack_device(dev, staging, dtype, layout, N, K, out);
    int st2 = mvlm_buffer_free(staging);
    return st != MVLM_OK ? st : st2;
}

extern "C" int mvlm_weight_free(mvlm_weight* w) {
    REQUIRE(w, "mvlm_weight_free: w is null");
    (void)hipSetDevice(w->dev->ordinal);
    int st = check_hip(hipFree(w->alloc), "hipFree(weight)");
    delete w;
    return st;
}

extern "C" int mvlm_weight_dtype(const mvlm_weight* w) { return w ? w->dtype : MVLM_ERR_INVALID_ARG; }

extern "C" int mvlm_weight_shape(const mvlm_weight* w, int* N, int* K) {
    REQUIRE(w && N && K, "mvlm_weight_shape: null argument");
    *N = w->N; *K = w->K;
    return MVLM_OK;
}

extern "C" size_t mvlm_weight_bytes(const mvlm_weight* w) { return w ? w->bytes : 0; }

extern "C" int mvlm_weight_dequant(mvlm_device* dev, const mvlm_weight* w, mvlm_buffer* out, mvlm_event** ev) {
    REQUIRE(dev && w && out, "mvlm_weight_dequant: null argument");
    REQUIRE(w->dev == dev && out->dev == dev, "mvlm_weight_dequant: handles belong to another device");
    size_t need = (size_t)w->N * (size_t)w->K * 4;
    if (out->bytes < need)
        return set_error(MVLM_ERR_BUFFER_TOO_SMALL, "mvlm_weight_dequant: output holds %zu bytes, %zu needed", out->bytes, need);
    LaunchScope ls(dev, ev);
    if (ls.status != MVLM_OK) return ls.status;
    hipError_t e = launch_dequant(dev->stream, w, (float*)out->ptr);
    if (e != hipSuccess) ls.status = check_hip(e, "dequant kernel");
    return ls.finish("dequant kernel");
}

extern "C" int mvlm_weight_random(mvlm_device* dev, int dtype, int N, int K, uint64_t seed,
                                  double wstd, mvlm_weight** out) {
    REQUIRE(dev && out, "mvlm_weight_random: null argument");
    *out = nullptr;
    REQUIRE(is_quant(dtype) || is_dense(dtype), "mvlm_weight_random: unsupported dtype %d", dtype);
    mvlm_weight* w = nullptr;
    int st = weight_alloc(dev, dtype, N, K, &w);
    if (st != MVLM_OK) return st;
    st = check_hip(launch_weight_random(dev->stream, w, seed, wstd), "weight_random kernel");
    if (st == MVLM_OK) st = check_hip(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
    if (st != MVLM_OK) { (void)hipFree(w->alloc); delete w; return st; }
    *out = w;
    return MVLM_OK;
}

extern "C" int mvlm_fill_normal(mvlm_device* dev, mvlm_buffer* buf, int dtype, size_t count,
                                uint64_t seed, double stddev) {
    REQUIRE(dev && buf, "mvlm_fill_normal: null argument");
    REQUIRE(is_dense(dtype), "mvlm_fill_normal: dtype %d is not F32/F16/BF16", dtype);
    if (count * dtype_size(dtype) > buf->bytes)
        return set_error(MVLM_ERR_BUFFER_TOO_SMALL, "mvlm_fill_normal: %zu elements do not fit %zu bytes", count, buf->bytes);
    if (count == 0) return MVLM_OK;
    HIP_TRY(launch_fill_normal(dev->stream, buf->ptr, dtype, count, seed, stddev));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    return MVLM_OK;
}

// ---------------------------------------------------------------------------
// events and markers
// ---------------------------------------------------------------------------

extern "C" int mvlm_event_wait(mvlm_event* ev) {
    REQUIRE(ev, "mvlm_event_wait: ev is null");
    HIP_TRY(hipEventSynchronize(ev->end ? ev->end : ev->start));
    return MVLM_OK;
}

extern "C" int mvlm_event_elapsed_ms(mvlm_event* ev, float* ms) {
    REQUIRE(ev && ms, "mvlm_event_elapsed_ms: null argument");
    REQUIRE(ev->start && ev->end, "mvlm_event_elapsed_ms: event is a single marker");
    HIP_TRY(hipEventSynchronize(ev->end));
    HIP_TRY(hipEventElapsedTime(ms, ev->start, ev->end));
    return MVLM_OK;
}

extern "C" int mvlm_event_release(mvlm_event* ev) {
    REQUIRE(ev, "mvlm_event_release: ev is null");
    int st = MVLM_OK;
    if (ev->start) st = check_hip(hipEventDestroy(ev->start), "hipEventDestroy");
    if (ev->end) { int s = check_hip(hipEventDestroy(ev->end), "hipEventDestroy"); if (st == MVLM_OK) st = s; }
    delete ev;
    return st;
}

extern "C" int mvlm_marker_record(mvlm_device* dev, mvlm_event** out) {
    REQUIRE(dev && out, "mvlm_marker_record: null argument");
    *out = nullptr;
    mvlm_event* ev = new (std::nothrow) mvlm_event();
    if (!ev) return set_error(MVLM_ERR_OUT_OF_MEMORY, "event allocation failed");
    ev->dev = dev;
    int st = check_hip(hipEventCreate(&ev->start), "hipEventCreate");
    if (st == MVLM_OK) st = check_hip(hipEventRecord(ev->start, dev->stream), "hipEventRecord");
    if (st != MVLM_OK) { if (ev->start) (void)hipEventDestroy(ev->start); delete ev; return st; }
    *out = ev;
    return MVLM_OK;
}

extern "C" int mvlm_marker_elapsed_ms(mvlm_event* start, mvlm_event* end, float* ms) {
    REQUIRE(start && end && ms, "mvlm_marker_elapsed_ms: null argument");
    HIP_TRY(hipEventSynchronize(end->start));
    HIP_TRY(hipEventElapsedTime(ms, start->start, end->start));
    return MVLM_OK;
}
