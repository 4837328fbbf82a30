// Internal definitions shared by the host runtime and the kernel files.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>

#include <utility>
#include <vector>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/mvlm_hip.h"

struct mvlm_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    hipDeviceProp_t prop{};
    // Workspace for ops that hand partial results between two launches (split
    // attention).  Grow-only: a larger request allocates a new block and keeps
    // the old ones, so a pointer an op (or a captured graph) holds stays valid
    // until the device is destroyed.  Ops on the device's one stream run in
    // order, so they share the current block.
    std::vector<void*> scratch_blocks;
    size_t scratch_bytes = 0;
    // Device address of the library's fixed workspace array on this GPU
    // (MVLM_NOALLOC_SCRATCH_BYTES, noalloc.hip), used only by the entry points
    // that allocate nothing; resolved at device creation.
    void* noalloc_scratch = nullptr;
    // Words of self-resetting cross-workgroup protocols (the split token
    // pick's per-row best key and arrival count): zero between launches, each
    // launch's last workgroup setting its words back.  Ops of one handle run in
    // order on its stream, so they never share a word.  Allocated and zeroed
    // at the first op that needs them.
    void* sync_words = nullptr;
};
constexpr int ARGMAX_SYNC_ROWS = 64;                                   // rows of split token picks
constexpr size_t SYNC_WORDS_BYTES = ARGMAX_SYNC_ROWS * (8 + 4);

struct mvlm_buffer {
    mvlm_device* dev = nullptr;
    void* ptr = nullptr;
    size_t bytes = 0;
    bool owned = false;        // false for views
    mvlm_buffer* parent = nullptr;
    int views = 0;             // live views of this buffer
};

// HBM layout of a packed weight, always [N][K] with K contiguous:
//  dense (F32/F16/BF16): data = [N][ld] elements, ld = K rounded up to 64,
//                        columns K..ld-1 zero.
//  Q8_0: data = int8 codes [N][K] (row stride K bytes);
//        scales = fp16 d [N][K/32].
//  Q4_0: data = nibble codes [N][K/2] (row stride K/2 bytes); each block of
//        32 weights is 16 bytes where byte j holds weight j in its low nibble
//        and weight j+16 in its high nibble (the GGUF order);
//        scales = fp16 d [N][K/32].
struct mvlm_weight {
    mvlm_device* dev = nullptr;
    int dtype = 0;
    int N = 0, K = 0;
    int64_t ld = 0;            // dense: elements per row; quant: code bytes per row
    void* data = nullptr;
    void* scales = nullptr;
    void* alloc = nullptr;     // single allocation holding data (+ scales)
    size_t bytes = 0;
};

struct mvlm_event {
    mvlm_device* dev = nullptr;
    hipEvent_t start = nullptr;
    hipEvent_t end = nullptr;
};

struct mvlm_pool {
    mvlm_buffer* buffers[2] = {nullptr, nullptr};
    size_t size = 0;
    int current = 0;
};

namespace mvlm {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_hip(hipError_t e, const char* what);

#define REQUIRE(cond, ...)                                                      \
    do {                                                                        \
        if (!(cond)) return ::mvlm::set_error(MVLM_ERR_INVALID_ARG, __VA_ARGS__); \
    } while (0)

#define HIP_TRY(expr)                                     \
    do {                                                  \
        int _st = ::mvlm::check_hip((expr), #expr);       \
        if (_st != MVLM_OK) return _st;                   \
    } while (0)

inline size_t dtype_size(int dt) {
    switch (dt) {
        case MVLM_F32: return 4;
        case MVLM_F16: case MVLM_BF16: return 2;
        default: return 0;
    }
}
inline bool is_dense(int dt) { return dt == MVLM_F32 || dt == MVLM_F16 || dt == MVLM_BF16; }
inline bool is_quant(int dt) { return dt == MVLM_Q8_0 || dt == MVLM_Q4_0; }
inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Device workspace of at least `bytes` (see mvlm_device::scratch_blocks).
int device_scratch(mvlm_device* dev, size_t bytes, void** out);
// The device's sync words (mvlm_device::sync_words), zeroed when first allocated.
int device_sync_words(mvlm_device* dev, void** out);
// Looks up the fixed workspace array's address on the current device
// (noalloc.hip); sets dev->noalloc_scratch.
int resolve_noalloc_scratch(mvlm_device* dev);

// Launch bracketing: records the start marker when the caller asked for an
// event, and finishes (end marker + hand-over) after the launch.
struct LaunchScope {
    mvlm_device* dev;
    mvlm_event** out;
    mvlm_event* ev = nullptr;
    int status = MVLM_OK;
    LaunchScope(mvlm_device* d, mvlm_event** o);
    int finish(const char* kernel_name);
};

// Every op enqueues exactly one kernel through launch_kernel.  When a caller
// sets kernel_timing (plan profiling), the launch carries start/stop events on
// its own dispatch packet (hipExtLaunchKernelGGL), which time the kernel's
// execution without adding marker packets between launches.
struct KernelTiming {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};
KernelTiming& kernel_timing();

template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t s,
                          Args&&... args) {
    KernelTiming& t = kernel_timing();
    if (t.start)
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, t.start, t.stop, 0, std::forward<Args>(args)...);
    else
        hipLaunchKernelGGL(kernel, grid, block, shmem, s, std::forward<Args>(args)...);
}

// Raises kernel Kernel's dynamic LDS limit to `bytes` on the current device,
// once per device and kernel; returns that call's status.  Concurrent first
// calls may both set the attribute, which is harmless.
template <auto Kernel>
inline hipError_t allow_dynamic_lds(int bytes) {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> status[kMaxDevices];   // 0: not set yet, else hipError_t + 1
    int dev = 0;
    if (const hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    auto set = [&] { return hipFuncSetAttribute((const void*)Kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes); };
    if (dev < 0 || dev >= kMaxDevices) return set();
    int st = status[dev].load(std::memory_order_acquire);
    if (st == 0) {
        st = (int)set() + 1;
        status[dev].store(st, std::memory_order_release);
    }
    return (hipError_t)(st - 1);
}

// An op made of two dependent kernels: the first carries the start event and
// the second the stop event, so plan profiling times the pair.
enum class LaunchPart { First, Middle, Last };
template <typename... KArgs, typename... Args>
inline void launch_kernel_part(LaunchPart part, void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem,
                               hipStream_t s, Args&&... args) {
    KernelTiming& t = kernel_timing();
    hipEvent_t start = part == LaunchPart::First ? t.start : nullptr;
    hipEvent_t stop = part == LaunchPart::Last ? t.stop : nullptr;
    if (t.start)
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, start, stop, 0, std::forward<Args>(args)...);
    else
        hipLaunchKernelGGL(kernel, grid, block, shmem, s, std::forward<Args>(args)...);
}

// Fused epilogue of a GEMM / GEMV store (mvlm_epilogue in mvlm_hip.h):
// out = act(acc + bias[n]) * mul[i] + res[i], i the output element's index;
// bias, mul and res have the output's dtype.
struct Epilogue {
    const void* bias = nullptr;
    const void* mul = nullptr;
    const void* res = nullptr;
    int act = 0;
    int dtype = 0;
    __host__ __device__ bool any() const { return bias || mul || res || act; }
};

// Kernel launchers (defined in the .hip files).  They assume validated input.
// A null Epilogue pointer means none.
hipError_t launch_gemm_naive(hipStream_t s, const uint16_t* A, const uint16_t* B, uint16_t* C,
                             int M, int N, int K);
hipError_t launch_gemm_tiled(hipStream_t s, const uint16_t* A, const uint16_t* B, uint16_t* C,
                             int M, int N, int K);
// y[N] = W[N,K] x[K], packed fp16 W, fp16 x and y, the reference gemv's
// summation order (x 8-byte aligned)
hipError_t launch_gemv_exact(hipStream_t s, const uint16_t* x, const mvlm_weight* W, uint16_t* y);
hipError_t launch_gemv_dense(hipStream_t s, const void* x, int x_dtype, const mvlm_weight* W,
                             void* y, int y_dtype, int N, int K, const Epilogue* ep = nullptr);
// Q8_0 / Q4_0 skinny GEMM on the matrix cores, 1 <= M <= 16 (any row length)
hipError_t launch_gemm_skinny(hipStream_t s, const float* X, const mvlm_weight* W, float* Y, int M, int N, int K,
                              int num_cus, const Epilogue* ep = nullptr);
// whether one skinny launch over these weights fits: K a multiple of 32 and,
// for the tile shape the launch would pick, the LDS (which stages all of a
// block's row-group scales) within the limit
bool skinny_supported(int count, const mvlm_weight* const* ws, int num_cus);
// M == 1 streaming GEMV for every weight format (rows of at most 16 KiB), and
// for quantized weights 2 <= M <= 4 rows of x (launch_gemv_stream_batch).
bool stream_supported(const mvlm_weight* w, int M = 1);
hipError_t launch_gemv_stream_batch(hipStream_t s, const float* x, const mvlm_weight* W, float* y, int M,
                                    int num_cus, const Epilogue* ep = nullptr);
hipError_t launch_gemv_stream(hipStream_t s, const void* x, int x_dtype, const mvlm_weight* W, void* y,
                              int y_dtype, int num_cus, const Epilogue* ep = nullptr);
// One launch for up to 8 independent problems of one weight dtype and x dtype;
// M > 1 (quantized weights, fp32 x and y, M <= 4) streams each weight once for
// its M rows of x.
struct StreamAttnDesc;
hipError_t launch_gemv_stream_group(hipStream_t s, int count, const void* const* xs, int x_dtype,
                                    const mvlm_weight* const* ws, void* const* ys, const int* y_dtypes, int num_cus,
                                    const Epilogue* eps = nullptr, int M = 1, const StreamAttnDesc* at = nullptr);
// Decode attention carried by an M = 1 grouped launch (gemv_stream.hip): one
// query per head against the KV cache (fp16 K and V [.][heads][D], D = 64 or
// 128), fp32 output o [heads][D].  step == 0: fp16 q [heads][D], `cached`
// keys.  step != 0: q, the new key and the new value are the three fp32
// thirds of qkv [3][heads][D]; they are rounded to fp16, the new key and
// value written to cache row `cached`, and q attends over cached + 1 keys.
// mode 0: the attention runs in the launch's first workgroups and the
// problems with x == o wait for it; mode 1 (step only): qkv is the output of
// one problem of the launch (N = 3 heads D) and the attention runs after that
// problem's rows are written.
struct StreamAttnDesc {
    const void* q = nullptr;
    const void* qkv = nullptr;
    void* k = nullptr;
    void* v = nullptr;
    float* o = nullptr;
    int heads = 0, head_dim = 0, cached = 0, mode = 0, step = 0;
    float scale = 0.0f;
    void* workspace = nullptr;     // stream_attn_workspace_bytes(heads, head_dim, cached, step, CUs)
    void* sync = nullptr;          // SYNC_BYTES of the launch site, zeroed before its first launch
};
constexpr size_t SYNC_BYTES = 64 * 1024;
constexpr size_t SYNC_ERR_OFFSET = 256;   // u32 error word of a sync area
size_t stream_attn_workspace_bytes(int heads, int head_dim, int cached, int step, int num_cus);
// hipSuccess when this launch can carry the attention: M = 1, head_dim 64 or
// 128, mode 0 with fp32 x and rows of at most 4 KiB for the waiting problems,
// mode 1 with one fp32 problem output equal to qkv, and the workgroups that
// wait unable to fill the device by themselves
hipError_t stream_attn_check(int count, const void* const* xs, int x_dtype, const mvlm_weight* const* ws,
                             void* const* ys, const int* y_dtypes, const StreamAttnDesc& at, int num_cus);
// The same attention as launches of its own (no sync area needed).
hipError_t launch_attn_decode(hipStream_t s, const StreamAttnDesc& d, int num_cus);
// Skinny GEMM over up to 8 independent problems (quantized weights of one
// dtype, fp32 X [M][K] and Y [M][N] each, 1 <= M <= 16) in one launch.
hipError_t launch_gemm_skinny_group(hipStream_t s, int M, int count, const float* const* Xs,
                                    const mvlm_weight* const* ws, float* const* Ys, int num_cus,
                                    const Epilogue* eps = nullptr);
inline int64_t weight_row_bytes(const mvlm_weight* w) { return is_dense(w->dtype) ? w->ld * (int64_t)dtype_size(w->dtype) : w->ld; }
// MFMA GEMM.  Its workspace (gemm_workspace_bytes) holds the fp32 partials
// of a K split (chosen by the launcher's cost model) and zero-padded copies of
// A and B when their rows are not 16-byte aligned: K, a leading dimension or
// a batch stride not a multiple of 8 elements, or B rows readable only up to
// kread_b < K rounded up to 8.
size_t gemm_workspace_bytes(int batch, int M, int N, int K, int64_t lda, int64_t ldb, int64_t sA, int64_t sB,
                            int kread_b, int num_cus);
// Batched NT products with K <= 128 (a multiple of 8) and a dense fp32 C per
// batch (ldc == N <= 1024), A/B/C 16-byte aligned: C's rows in blocks of 16,
// each written as one contiguous range (gemm_smallk.hip).
bool smallk_supported(int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA, int64_t sB,
                      const void* A, const void* B, const void* C);
hipError_t launch_gemm_smallk(hipStream_t s, const void* A, int ab_dtype, const void* B, float* C, int batch, int M,
                              int N, int K, int64_t lda, int64_t ldb, int64_t sA, int64_t sB, int64_t sC, int num_cus);
hipError_t launch_gemm_mfma(hipStream_t s, const void* A, int ab_dtype, const void* B, void* C,
                            int c_dtype, int batch, int M, int N, int K, int64_t lda, int64_t ldb,
                            int64_t ldc, int64_t strideA, int64_t strideB, int64_t strideC,
                            int kread_b, int num_cus, const Epilogue* ep, void* workspace, size_t workspace_bytes);
// fused attention, fp16 Q/K/V [seq][heads][head_dim], head_dim a multiple of 8 up to 128;
// `workspace` holds attention_workspace_bytes(...) bytes (none when that is 0)
size_t attention_workspace_bytes(int seq_q, int seq_kv, int heads, int head_dim, int num_cus);
hipError_t launch_attention(hipStream_t s, const void* Q, const void* K, const void* V, void* O, int o_dtype,
                            int seq_q, int seq_kv, int heads, int head_dim, int causal, float scale, int num_cus,
                            void* workspace, size_t workspace_bytes);
// row-wise argmax (first index of the largest key), one workgroup per row
// sync: the device's sync words (device_sync_words), or null for the
// one-workgroup-per-row form only
hipError_t launch_argmax(hipStream_t s, const void* x, int dtype, int rows, int n, int64_t ld, int* out,
                         void* sync = nullptr);
int argmax_splits(int rows, int n);
hipError_t launch_pack(hipStream_t s, const void* src, int dtype, int layout, int N, int K,
                       mvlm_weight* w);
hipError_t launch_dequant(hipStream_t s, const mvlm_weight* w, float* out);
hipError_t launch_fill_normal(hipStream_t s, void* dst, int dtype, size_t count, uint64_t seed,
                              double stddev);
hipError_t launch_weight_random(hipStream_t s, mvlm_weight* w, uint64_t seed, double wstd);

}  // namespace mvlm
