/*
 * mvlm_hip.h — C ABI of the MI355X (gfx950) matmul hot path of MVLM.
 *
 * Plain C: opaque handles, pointers and sizes; no HIP, OpenCL or C++ types.
 * Every function returns an int status (MVLM_OK == 0, negative on error); on
 * error it also prints the message to stderr (as the reference's CL_CHECK_NULL
 * does, src/engine/compute.cpp:12-17) and keeps it for mvlm_last_error().
 *
 * Layout contract.  Packed weights are built from either
 *   - MVLM_LAYOUT_NK: GGUF-native [N rows][K], K contiguous (y = x * W^T), or
 *   - MVLM_LAYOUT_KN: the reference's create_weight_image input, [K rows][N]
 *     (src/engine/memory.cpp:28-79, rows = K, cols = N),
 * and always hold the weight as [N][K] in HBM.  Quantized weights (Q8_0, Q4_0)
 * are accepted only as GGUF blocks along K (MVLM_LAYOUT_NK, K % 32 == 0).
 *
 * Threading.  One in-order HIP stream per device handle, default priority.
 * Calls on one handle are not thread-safe (as the reference's single in-order
 * queue, src/engine/device.cpp:298-300).  Launch functions only enqueue; an
 * mvlm_event** argument may be NULL, otherwise the caller owns the returned
 * event and releases it with mvlm_event_release (src/engine/compute.cpp
 * returns a cl_event the caller must wait on and release).
 */
#ifndef MVLM_HIP_H
#define MVLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MVLM_ABI_VERSION 3

/* ---- status codes ------------------------------------------------------- */
enum mvlm_status {
    MVLM_OK = 0,
    MVLM_ERR_INVALID_ARG = -1,   /* null handle, bad size, bad dtype/layout  */
    MVLM_ERR_NO_DEVICE = -2,     /* no HIP device, or ordinal out of range   */
    MVLM_ERR_OUT_OF_MEMORY = -3, /* device or host allocation failed        */
    MVLM_ERR_HIP = -4,           /* a HIP runtime call failed               */
    MVLM_ERR_UNSUPPORTED = -5,   /* valid request this library does not serve */
    MVLM_ERR_BUFFER_TOO_SMALL = -6,
    MVLM_ERR_NOT_FOUND = -7,     /* no such tensor / metadata key            */
    MVLM_ERR_FORMAT = -8         /* malformed or truncated file              */
};

/* ---- element types (ggml type ids, src/models/gguf_loader.h:12-31) ----- */
enum mvlm_dtype {
    MVLM_F32 = 0,
    MVLM_F16 = 1,
    MVLM_Q4_0 = 2,
    MVLM_Q8_0 = 8,
    MVLM_BF16 = 30
};

enum mvlm_layout { MVLM_LAYOUT_NK = 0, MVLM_LAYOUT_KN = 1 };

typedef struct mvlm_device mvlm_device;
typedef struct mvlm_buffer mvlm_buffer;
typedef struct mvlm_weight mvlm_weight;
typedef struct mvlm_event mvlm_event;
typedef struct mvlm_pool mvlm_pool;

/* Mirrors the fields of the reference's DeviceInfo that make sense on HIP
 * (src/engine/device.h:13-55) plus the peaks used for roofline fractions. */
typedef struct mvlm_device_info {
    char device_name[256];
    char arch_name[64];              /* e.g. "gfx950:sramecc+:xnack-" */
    int ordinal;
    int compute_units;
    int max_clock_mhz;
    int memory_clock_mhz;
    int memory_bus_width_bits;
    int wavefront_size;
    uint64_t global_mem_size;
    uint64_t local_mem_size;         /* LDS bytes per work-group */
    uint64_t l2_cache_size;
    double peak_hbm_gbs;             /* nominal MI355X HBM3E: 8000 GB/s */
    double peak_fp16_tflops;         /* nominal dense fp16/bf16 MFMA: 2500 */
    /* the same peaks derived from this device's reported properties, as the
     * reference bench derives its peak (gemm_bench.cpp:180-182): CUs x clock x
     * 4096 dense fp16 flops per CU per clock (4 SIMDs of CDNA4), and memory
     * clock x bus width x 4 / 8 (HBM3E: data on both edges of a write clock
     * running at twice the reported memory clock) */
    double box_peak_hbm_gbs;
    double box_peak_fp16_tflops;
} mvlm_device_info;

/* ---- errors -------------------------------------------------------------- */
/* Message of the last failing call on this thread ("" if none). */
const char* mvlm_last_error(void);
int mvlm_abi_version(void);

/* ---- device lifecycle (src/engine/device.h:58-75) ------------------------ */
int mvlm_device_count(int* count);
/* replaces init_device (device.cpp:141-304); no program build step: the
 * gfx950 code objects are part of this library. */
int mvlm_device_create(int ordinal, mvlm_device** out);
int mvlm_device_destroy(mvlm_device* dev);                      /* destroy_device */
int mvlm_device_get_info(const mvlm_device* dev, mvlm_device_info* info);
int mvlm_device_synchronize(mvlm_device* dev);                  /* clFinish */

/* ---- buffers (src/engine/memory.h:15-35) ---------------------------------- */
/* create_buffer (memory.cpp:81-89): device allocation of `bytes`. */
int mvlm_buffer_alloc(mvlm_device* dev, size_t bytes, mvlm_buffer** out);
/* A view of [offset, offset+bytes) of `parent` (the reference makes a
 * sub-buffer for the last row before the LM head, moondream2.cpp:528-536).
 * The view must be freed before its parent. */
int mvlm_buffer_view(mvlm_buffer* parent, size_t offset, size_t bytes, mvlm_buffer** out);
int mvlm_buffer_free(mvlm_buffer* buf);
size_t mvlm_buffer_size(const mvlm_buffer* buf);
/* Synchronous host<->device copies on the device stream. */
int mvlm_buffer_upload(mvlm_buffer* buf, size_t offset, const void* src, size_t bytes);
int mvlm_buffer_download(const mvlm_buffer* buf, size_t offset, void* dst, size_t bytes);
int mvlm_buffer_fill_zero(mvlm_buffer* buf);

/* BufferPool ping-pong (memory.h:25-35, memory.cpp:113-157). */
int mvlm_pool_init(mvlm_device* dev, size_t bytes, mvlm_pool** out);   /* init_buffer_pool */
mvlm_buffer* mvlm_pool_current(mvlm_pool* pool);                       /* get_current_buffer */
mvlm_buffer* mvlm_pool_next(mvlm_pool* pool);                          /* get_next_buffer */
int mvlm_pool_swap(mvlm_pool* pool);                                   /* swap_buffers */
int mvlm_pool_destroy(mvlm_pool* pool);                                /* destroy_buffer_pool */

/* ---- packed weights (replaces create_weight_image, memory.cpp:28-79) ---- */
/* `src` is host memory: for F32/F16/BF16 N*K elements in `layout`; for Q8_0 /
 * Q4_0 N*(K/32) GGUF blocks (34 / 18 bytes) in MVLM_LAYOUT_NK. */
int mvlm_weight_pack(mvlm_device* dev, const void* src, int dtype, int layout,
                     int N, int K, mvlm_weight** out);
/* Same, from GGUF-layout bytes already in device memory (no host staging). */
int mvlm_weight_pack_device(mvlm_device* dev, const mvlm_buffer* src, int dtype, int layout,
                            int N, int K, mvlm_weight** out);
int mvlm_weight_free(mvlm_weight* w);
int mvlm_weight_dtype(const mvlm_weight* w);
int mvlm_weight_shape(const mvlm_weight* w, int* N, int* K);
/* Bytes the weight occupies in HBM (codes + scales + padding). */
size_t mvlm_weight_bytes(const mvlm_weight* w);
/* Writes the exact fp32 values of the packed weight as [N][K] row-major into
 * `out` (N*K*4 bytes): d*q for Q8_0, (q-8)*d for Q4_0. */
int mvlm_weight_dequant(mvlm_device* dev, const mvlm_weight* w, mvlm_buffer* out, mvlm_event** ev);

/* ---- reference GEMM entry points (src/engine/compute.h:13-33) ------------ */
/* C[M,N] = A[M,K] * B[K,N]; A, B, C fp16 row-major, fp32 accumulation in
 * ascending k with fused multiply-add, round-to-nearest-even fp16 store: the
 * arithmetic of gemm_naive (gemm.cl:26-51).  dispatch_gemm_naive. */
int mvlm_gemm_naive(mvlm_device* dev, const mvlm_buffer* A, const mvlm_buffer* B,
                    mvlm_buffer* C, int M, int N, int K, mvlm_event** ev);
/* Same arithmetic as gemm_tiled (gemm.cl:74-136), LDS-tiled; bit-identical
 * to mvlm_gemm_naive.  dispatch_gemm_tiled. */
int mvlm_gemm_tiled(mvlm_device* dev, const mvlm_buffer* A, const mvlm_buffer* B,
                    mvlm_buffer* C, int M, int N, int K, mvlm_event** ev);
/* dispatch_gemm_image (compute.cpp:90-120): C[M,N] = A[M,K] * W, W a packed
 * weight (F16 or BF16), computed on MFMA with fp32 accumulation.  a_dtype is
 * F16 or BF16 (matching W), c_dtype F32, F16 or BF16. */
int mvlm_gemm_packed(mvlm_device* dev, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                     mvlm_buffer* C, int c_dtype, int M, int N, int K, mvlm_event** ev);
/* dispatch_gemv (compute.cpp:122-152): y[N] = x[K] * W.  W packed F32, F16,
 * BF16, Q8_0 or Q4_0; x_dtype F32, F16 or BF16 (F32 for quantized W);
 * y_dtype F32, F16 or BF16.  fp32 accumulation. */
int mvlm_gemv(mvlm_device* dev, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W,
              mvlm_buffer* y, int y_dtype, int N, int K, mvlm_event** ev);
/* dispatch_gemv (compute.cpp:122-152) with the arithmetic of gemv
 * (gemm.cl:215-270): y[N] = x[K] * W for a packed F16 weight, fp16 x (8-byte
 * aligned) and fp16 y; each output is 256 fp32 fma partials over
 * k = L, L+256, ..., folded pairwise over strides 128..1 and stored
 * round-to-nearest-even, so y is bit-identical to the reference's.
 * mvlm_gemv is the faster path for the same product. */
int mvlm_gemv_exact(mvlm_device* dev, const mvlm_buffer* x, const mvlm_weight* W, mvlm_buffer* y,
                    int N, int K, mvlm_event** ev);

/* ---- fused epilogues ----------------------------------------------------------
 * out = act(acc + bias[n]) * mul[m][n] + residual[m][n], applied to the fp32
 * accumulator before the output is rounded to its dtype, so the bias add,
 * activation, gate product and residual add of a transformer block cost no
 * extra pass over HBM.  Replaces the separate kernels the reference runs
 * after its projections: bias adds (vision.cl:178-186, 433-436), gelu
 * (activations.cl:66-118), silu / silu_gate_multiply (activations.cl:22-60,
 * 204-255) and vector_add for residuals (activations.cl:259-290).
 * MVLM_ACT_GELU_TANH is 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), the
 * formula of activations.cl:68 (the kernel there evaluates the tanh with the
 * sign flipped, activations.cl:96-116, which this library does not reproduce).
 * bias ([N]), mul and residual ([M][N], row stride N) are optional, have the
 * output's dtype, start at a multiple of its size (else MVLM_ERR_INVALID_ARG),
 * and may alias the output. */
enum mvlm_activation {
    MVLM_ACT_NONE = 0,
    MVLM_ACT_GELU_TANH = 1,
    MVLM_ACT_SILU = 2          /* x / (1 + exp(-x)) */
};
typedef struct mvlm_epilogue {
    const mvlm_buffer* bias;
    int activation;
    const mvlm_buffer* mul;
    const mvlm_buffer* residual;
} mvlm_epilogue;
/* mvlm_gemm_packed / mvlm_gemv with an epilogue (NULL = none).  For
 * quantized W the epilogue applies at M == 1 (mvlm_gemv_ex). */
int mvlm_gemm_packed_ex(mvlm_device* dev, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                        mvlm_buffer* C, int c_dtype, int M, int N, int K, const mvlm_epilogue* ep,
                        mvlm_event** ev);
int mvlm_gemv_ex(mvlm_device* dev, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W,
                 mvlm_buffer* y, int y_dtype, int N, int K, const mvlm_epilogue* ep, mvlm_event** ev);

/* mvlm_gemm_packed_ex without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * workspace (K-split partials, zero-padded copies of A when K % 8 != 0) comes
 * from one fixed device array of MVLM_NOALLOC_SCRATCH_BYTES per GPU, reserved
 * by the library for the life of the process; a shape that needs more is
 * refused with MVLM_ERR_UNSUPPORTED.  Results are identical to
 * mvlm_gemm_packed_ex's.  All calls on one GPU share the array: calls through
 * one device handle run in order on its stream, calls that overlap on one GPU
 * (several handles or streams) race.  No event is returned. */
#define MVLM_NOALLOC_SCRATCH_BYTES (32u << 20)
int mvlm_gemm_packed_ex_noalloc(mvlm_device* dev, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                                mvlm_buffer* C, int c_dtype, int M, int N, int K, const mvlm_epilogue* ep);

/* ---- grouped decode GEMV ----------------------------------------------------
 * Up to MVLM_MAX_GROUP independent GEMVs (M = 1) in one launch, e.g. the
 * projections of one Phi-1.5 block that do not depend on each other: QKV and
 * fc1 read the same input, dense and fc2 read the attention and MLP branches.
 * The reference issues them as separate dispatch_gemv calls
 * (src/models/moondream2.cpp:374-508).  All weights share one dtype and all
 * x one dtype; each entry has the arguments and checks of mvlm_gemv. */
#define MVLM_MAX_GROUP 8
typedef struct mvlm_gemv_desc {
    const mvlm_buffer* x;
    int x_dtype;
    const mvlm_weight* W;
    mvlm_buffer* y;
    int y_dtype;
} mvlm_gemv_desc;
int mvlm_gemv_grouped(mvlm_device* dev, int count, const mvlm_gemv_desc* descs, mvlm_event** ev);
/* The same grouping for M rows of activations over Q8_0 / Q4_0 weights
 * (batched decode; the reference has no batched path): each entry is
 * Y[M,N] = X[M,K] * W^T with fp32 X and Y and the checks of mvlm_gemm_q8_0 /
 * mvlm_gemm_q4_0, 1 <= M <= 16, one weight dtype for all entries. */
int mvlm_gemm_quant_grouped(mvlm_device* dev, int M, int count, const mvlm_gemv_desc* descs, mvlm_event** ev);
/* The grouped launches with a fused epilogue per entry: eps[i] (NULL = no
 * epilogue for any entry) is applied to entry i's output as in mvlm_gemv_ex,
 * with bias [N_i] and mul / residual [M][N_i] in entry i's y dtype.  This fuses
 * the bias, GELU and residual adds around the projections of one block
 * (moondream2.cpp:369-509; activations.cl:66-118, 259-290) into the launch. */
int mvlm_gemv_grouped_ex(mvlm_device* dev, int count, const mvlm_gemv_desc* descs, const mvlm_epilogue* eps,
                         mvlm_event** ev);
int mvlm_gemm_quant_grouped_ex(mvlm_device* dev, int M, int count, const mvlm_gemv_desc* descs,
                               const mvlm_epilogue* eps, mvlm_event** ev);

/* ---- dequantizing GEMV / skinny GEMM (planned in README.md:57, PLAN.md:65) */
/* y[N] = x[K] * W^T, W packed Q8_0, x and y fp32. */
int mvlm_gemv_q8_0(mvlm_device* dev, const mvlm_buffer* x, const mvlm_weight* W,
                   mvlm_buffer* y, int N, int K, mvlm_event** ev);
int mvlm_gemv_q4_0(mvlm_device* dev, const mvlm_buffer* x, const mvlm_weight* W,
                   mvlm_buffer* y, int N, int K, mvlm_event** ev);
/* Y[M,N] = X[M,K] * W^T for 1 <= M <= 16, X and Y fp32 row-major. */
int mvlm_gemm_q8_0(mvlm_device* dev, const mvlm_buffer* X, const mvlm_weight* W,
                   mvlm_buffer* Y, int M, int N, int K, mvlm_event** ev);
int mvlm_gemm_q4_0(mvlm_device* dev, const mvlm_buffer* X, const mvlm_weight* W,
                   mvlm_buffer* Y, int M, int N, int K, mvlm_event** ev);

/* ---- batched NT GEMM (the Q*K^T of attention.cl:84-88, all heads at once) */
/* C[b][m][n] = sum_k A[b][m][k] * B[b][n][k]; A, B fp16, C fp32; leading
 * dimensions and batch strides in elements. */
int mvlm_gemm_batched(mvlm_device* dev, const mvlm_buffer* A, const mvlm_buffer* B,
                      mvlm_buffer* C, int batch, int M, int N, int K,
                      int64_t lda, int64_t ldb, int64_t ldc,
                      int64_t strideA, int64_t strideB, int64_t strideC, mvlm_event** ev);

/* ---- fused attention (QK^T -> softmax -> PV in one kernel) ---------------
 * Q [seq_q][num_heads][head_dim], K and V [seq_kv][num_heads][head_dim], all
 * fp16 (the layout of attention.cl:44); O [seq_q][num_heads][head_dim] in
 * o_dtype (F16 or F32).  O = softmax(scale * Q K^T + mask) V per head, with
 * scale = 1/sqrt(head_dim) when scale == 0.  causal != 0 hides key k from
 * query q when k > q + (seq_kv - seq_q): queries are the last seq_q positions
 * of the keys (seq_q <= seq_kv required).  head_dim: a multiple of 8, at most
 * 128.  Scores and the softmax stay on chip (the 16 x 729 x 729 score tensor
 * of a SigLIP layer never reaches HBM). */
int mvlm_attention(mvlm_device* dev, const mvlm_buffer* Q, const mvlm_buffer* K,
                   const mvlm_buffer* V, mvlm_buffer* O, int o_dtype, int seq_q, int seq_kv,
                   int num_heads, int head_dim, int causal, float scale, mvlm_event** ev);
/* Replaces dispatch_attention_prefill (src/engine/compute.h:65,
 * compute.cpp:305-335; kernel attention.cl:46-179): causal attention of
 * seq_len queries over seq_len keys, scale 1/sqrt(head_dim), fp16 output. */
int mvlm_attention_prefill(mvlm_device* dev, const mvlm_buffer* Q, const mvlm_buffer* K,
                           const mvlm_buffer* V, mvlm_buffer* output, int seq_len, int num_heads,
                           int head_dim, mvlm_event** ev);
/* Replaces dispatch_attention_decode (src/engine/compute.h:70,
 * compute.cpp:337-367; kernel attention.cl:197-295): one query per head
 * ([1][num_heads][head_dim]) over cache_len cached keys, no mask, fp16 output. */
int mvlm_attention_decode(mvlm_device* dev, const mvlm_buffer* Q, const mvlm_buffer* K_cache,
                          const mvlm_buffer* V_cache, mvlm_buffer* output, int cache_len,
                          int num_heads, int head_dim, mvlm_event** ev);
/* One decode step of attention from the fused QKV projection's output, the
 * sequence of src/models/moondream2.cpp:404-440 without the rotary embedding:
 * kv_cache_append (moondream2.cpp:305-316, :419) then attention_decode
 * (attention.cl:197-295) over the grown cache.  qkv: fp32 [3][num_heads]
 * [head_dim] = q, the new key, the new value.  The new key and value are
 * rounded to fp16 (RNE) and written to row `cached` of K_cache / V_cache
 * (fp16 [cached + 1][num_heads][head_dim]); q, rounded to fp16, attends over
 * the cached + 1 keys with scale (1/sqrt(head_dim) when 0); O: fp32
 * [num_heads][head_dim].  head_dim 64 or 128, at most 192 heads.  In a plan,
 * right after the grouped GEMV that writes qkv, it runs inside that GEMV's
 * launch (see mvlm_plan_set_fusion). */
int mvlm_attention_decode_step(mvlm_device* dev, const mvlm_buffer* qkv, mvlm_buffer* K_cache,
                               mvlm_buffer* V_cache, mvlm_buffer* O, int cached, int num_heads,
                               int head_dim, float scale, mvlm_event** ev);

/* ---- token pick: row-wise argmax on the device ----------------------------
 * Replaces argmax_logits (src/models/moondream2.cpp:553-593), which reads the
 * fp16 logits back to the host and scans them.  out_index[r] (int32, device)
 * = the first index of the largest key of row r of x (rows x n, leading
 * dimension ld elements, dtype F32/F16/BF16).  Key: zeros and subnormals
 * count as 0, inf and NaN as +inf or -inf by their sign, other values as
 * themselves (the reference's fp16 decode, moondream2.cpp:571-583); a row of
 * -inf returns 0. */
int mvlm_argmax(mvlm_device* dev, const mvlm_buffer* x, int dtype, int rows, int n, int64_t ld,
                mvlm_buffer* out_index, mvlm_event** ev);

/* ---- synthetic inputs on the device ------------------------------------- */
/* SplitMix64 -> Box-Muller fills (same generator as the CPU oracle, computed
 * on the GPU so multi-GB weight sets need no host staging). */
int mvlm_fill_normal(mvlm_device* dev, mvlm_buffer* buf, int dtype, size_t count,
                     uint64_t seed, double stddev);
/* Random GGUF-distributed quantized weight, packed directly:
 * Q8_0 qs uniform in [-127,127], d = f16(|N(0,wstd)|/127);
 * Q4_0 codes uniform in [0,15],  d = f16(|N(0,wstd)|/8). */
int mvlm_weight_random(mvlm_device* dev, int dtype, int N, int K, uint64_t seed,
                       double wstd, mvlm_weight** out);

/* ---- events (src/engine/profiler.cpp:25-54 reads START/END of a cl_event) */
int mvlm_event_wait(mvlm_event* ev);
/* Device time between the launch's start and end markers, in ms. */
int mvlm_event_elapsed_ms(mvlm_event* ev, float* ms);
int mvlm_event_release(mvlm_event* ev);

/* ---- plans: a recorded sequence of launches -------------------------------
 * The decode-step driver.  The reference issues one dispatch per projection
 * and blocks on each event (src/models/moondream2.cpp:359-541, e.g. :379);
 * its "recordable queue" replay is an empty stub (src/engine/pipeline.cpp:45-125).
 * A plan records the launches once (validated at add time, like the direct
 * entry points), then enqueues them from native code, optionally replaying a
 * captured HIP graph.  Buffers and weights a plan names must outlive it. */
typedef struct mvlm_plan mvlm_plan;
int mvlm_plan_create(mvlm_device* dev, mvlm_plan** out);
int mvlm_plan_destroy(mvlm_plan* plan);
int mvlm_plan_size(const mvlm_plan* plan);
/* Y[M,N] = X[M,K] * W^T with N, K taken from W: dense W needs M == 1
 * (mvlm_gemv); Q8_0 / Q4_0 W takes 1 <= M <= 16 (mvlm_gemm_q8_0/q4_0). */
int mvlm_plan_add_gemv(mvlm_plan* plan, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W,
                       mvlm_buffer* y, int y_dtype, int M);
int mvlm_plan_add_gemv_grouped(mvlm_plan* plan, int count, const mvlm_gemv_desc* descs);
int mvlm_plan_add_gemm_quant_grouped(mvlm_plan* plan, int M, int count, const mvlm_gemv_desc* descs);
/* plan entries of mvlm_gemv_grouped_ex / mvlm_gemm_quant_grouped_ex */
int mvlm_plan_add_gemv_grouped_ex(mvlm_plan* plan, int count, const mvlm_gemv_desc* descs, const mvlm_epilogue* eps);
int mvlm_plan_add_gemm_quant_grouped_ex(mvlm_plan* plan, int M, int count, const mvlm_gemv_desc* descs,
                                        const mvlm_epilogue* eps);
/* plan entries with a fused epilogue (mvlm_gemv_ex, M == 1; mvlm_gemm_packed_ex) */
int mvlm_plan_add_gemv_ex(mvlm_plan* plan, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W,
                          mvlm_buffer* y, int y_dtype, const mvlm_epilogue* ep);
int mvlm_plan_add_gemm_packed_ex(mvlm_plan* plan, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                                 mvlm_buffer* C, int c_dtype, int M, const mvlm_epilogue* ep);
int mvlm_plan_add_gemm_packed(mvlm_plan* plan, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                              mvlm_buffer* C, int c_dtype, int M);
int mvlm_plan_add_gemm_batched(mvlm_plan* plan, const mvlm_buffer* A, const mvlm_buffer* B,
                               mvlm_buffer* C, int batch, int M, int N, int K,
                               int64_t lda, int64_t ldb, int64_t ldc,
                               int64_t strideA, int64_t strideB, int64_t strideC);
int mvlm_plan_add_attention(mvlm_plan* plan, const mvlm_buffer* Q, const mvlm_buffer* K,
                            const mvlm_buffer* V, mvlm_buffer* O, int o_dtype, int seq_q, int seq_kv,
                            int num_heads, int head_dim, int causal, float scale);
int mvlm_plan_add_attention_decode_step(mvlm_plan* plan, const mvlm_buffer* qkv, mvlm_buffer* K_cache,
                                        mvlm_buffer* V_cache, mvlm_buffer* O, int cached, int num_heads,
                                        int head_dim, float scale);
int mvlm_plan_add_argmax(mvlm_plan* plan, const mvlm_buffer* x, int dtype, int rows, int n, int64_t ld,
                         mvlm_buffer* out_index);
/* enable != 0: capture the plan into a HIP graph (now) and replay it on run. */
int mvlm_plan_use_graph(mvlm_plan* plan, int enable);
/* Enqueue the plan `repeats` times; `ev` (optional) spans everything enqueued. */
int mvlm_plan_run(mvlm_plan* plan, int repeats, mvlm_event** ev);
/* One eager run in which every launch carries start/stop events on its own
 * dispatch: op_ms[i] is the execution time of launch i (the figure
 * rocprofv3 --kernel-trace reports for that dispatch); an entry carried by
 * the next entry's launch (plan fusion) reports 0. */
int mvlm_plan_profile(mvlm_plan* plan, float* op_ms, int capacity);
/* Plan fusion.  No counterpart in the reference, whose decode loop launches
 * the projections, attention_decode and the output projection one by one
 * (src/models/moondream2.cpp:369-446).  A decode attention runs inside the
 * launch of a neighbouring grouped M == 1 GEMV entry:
 * (1) a decode attention step entry right after the grouped GEMV one of whose
 *     entries writes its qkv (F32, N = 3 num_heads head_dim): its workgroups
 *     follow that entry's, load their cached keys and values, and wait for
 *     the workgroups writing their head's rows; fused when no other entry
 *     writes qkv, the caches or O and no entry reads the caches or O;
 * (2) a decode attention entry (seq_q == 1, F32 output, head_dim 64 or 128)
 *     right before a grouped GEMV (F32 x) some of whose entries read its
 *     output as x: its workgroups come first, and the entries reading the
 *     output wait for it after loading their weights; fused when no entry
 *     writes the attention's inputs or output or reads the output other than
 *     as x, and the waiting entries have weight rows of at most 4 KiB in HBM
 *     (codes only for Q8_0 / Q4_0: K <= 4096 / 8192).
 * Either way the workgroups that wait must not be able to fill the device
 * alone; otherwise, or with fusion off, both entries launch as before.  The
 * pair is set up when the second entry is added.  On by default;
 * set_fusion(0) launches every entry separately (drops a captured graph).
 * mvlm_plan_fused returns the number of fused pairs in effect.
 * A waiting workgroup gives up after 20 ms and stores NaN;
 * mvlm_plan_check synchronizes and returns MVLM_ERR_HIP if a fused launch of
 * the plan gave up since the last check (and clears that launch site's
 * counters, so later runs start clean). */
int mvlm_plan_set_fusion(mvlm_plan* plan, int enable);
int mvlm_plan_fused(const mvlm_plan* plan);
int mvlm_plan_check(mvlm_plan* plan);

/* ---- stream markers for host-side timing of a region ---------------------- */
/* Records a marker on the device stream; elapsed time between two markers. */
int mvlm_marker_record(mvlm_device* dev, mvlm_event** out);
int mvlm_marker_elapsed_ms(mvlm_event* start, mvlm_event* end, float* ms);

/* ---- measurement of a design alternative --------------------------------- */
/* No counterpart in the reference.  Runs `rounds` (1..1000) software grid
 * barriers in one launch of one workgroup per CU, each preceded by a 256-byte
 * store and its wait, and reports the time per round: the cost a persistent
 * single-launch decode step would pay at each dependent stage, to compare with
 * a kernel boundary.  variant 0: one counter, returning atomic add, polls;
 * 1: one flag per workgroup, every workgroup polls all flags; 2: counter whose
 * last arriver raises a done flag replicated on 32 lines.  background != 0:
 * the workgroups' other 8 waves stream HBM meanwhile.  Waits are bounded
 * (20 ms); a wait that gives up returns MVLM_ERR_HIP.  Synchronous; allocates
 * (512 MiB with background). */
int mvlm_probe_grid_barrier(mvlm_device* dev, int variant, int rounds, int background, double* us_per_round);

/* Load latency at the start of a kernel (no counterpart in the reference: the
 * measurement behind the small-K product's loads).  One workgroup of 16 waves
 * per CU; each wave times one 16-byte-per-lane buffer load from its issue to
 * its return with s_memrealtime: variant 0 reads lines of a freshly written
 * 1 GiB buffer (from HBM), variant 1 an offset past the buffer's size (zeros,
 * no data moved); `after` (0, 4 or 9) more loads of the wave are issued behind
 * it.  us[0..3] = min, median, 90th percentile and max over the waves, in
 * microseconds.  Synchronous; allocates 1 GiB. */
int mvlm_probe_load_latency(mvlm_device* dev, int variant, int after, double* us);

#ifdef __cplusplus
}
#endif
#endif
