/*
 * oracle.h — CPU restatement of the MVLM matmul hot path (TEST INFRASTRUCTURE).
 *
 * This library is the checker, never the product: only the test suite, the
 * smoke check and the CPU-baseline leg of the benchmark may load it.  The
 * shipped library (libmvlm_hip.so) never links or calls it, and the HIP path
 * fails loudly when its own extension is missing instead of falling back here.
 *
 * What each function restates (paths relative to the reference repository):
 *   orc_gemm_naive   src/kernels/gemm.cl:26-51   (fp16 in, fp32 fma chain in
 *                    ascending k, vstore_half = RNE fp16 out)
 *   orc_gemm_tiled   src/kernels/gemm.cl:64-136  (8x8x8 local tiles, same k order)
 *   orc_gemm_image   src/kernels/gemm.cl:139-200 + src/engine/memory.cpp:28-79
 *                    (RGBA-half image, cols zero-padded to x4, 4 cols per item)
 *   orc_gemv         src/kernels/gemm.cl:215-270 + src/engine/compute.cpp:122-152
 *                    (256-lane strided partials, LDS tree 128..1, half4 store)
 *   orc_dequant_*    GGUF/ggml block definitions whose sizes the reference pins in
 *                    src/models/gguf_loader.cpp:13-55 and tests/test_gguf.cpp:16-34
 *                    (Q8_0: {fp16 d; int8 qs[32]}, Q4_0: {fp16 d; uint8 qs[16]}).
 *   orc_gemm_*_nk    the planned dequantizing / fp32 / fp16 GEMV-GEMM (README.md:57,
 *                    PLAN.md:65): dequantize exactly, then an fp32 fma chain in
 *                    ascending k, weights stored [N,K] as in GGUF.
 *   orc_*_f64        fp64 brute force plus the scale sum_k |a_k * b_k| used by the
 *                    tolerance |y - r| <= rtol * scale.
 *   orc_attention_f64  src/kernels/attention.cl:46-179 / :197-295 (softmax(Q K^T
 *                    / sqrt(d) + causal mask) V per head) in fp64.
 *   orc_argmax*      src/models/moondream2.cpp:553-593 (host argmax of the logits).
 *
 * Pinning (each function has at least one check that does not retype it):
 * golden fixtures under tests/golden/, closed forms (one-hot, identity,
 * exact-integer inputs where every order of summation agrees bit for bit),
 * numpy's float16 RNE conversion, fp64 brute force, and cross-checks between
 * restatements whose reference kernels share an fma order (naive == tiled ==
 * image bit for bit).
 */
#ifndef MVLM_ORACLE_H
#define MVLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats ---------------------------------------------------- */
uint16_t orc_f32_to_f16(float f);   /* round to nearest even, with subnormals and inf/nan */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);  /* round to nearest even */
float    orc_bf16_to_f32(uint16_t h);
void     orc_f32_to_f16_array(const float* src, uint16_t* dst, size_t n);
void     orc_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);
void     orc_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n);
void     orc_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* ---- seeded inputs: SplitMix64 -> Box-Muller (fp64) -------------------- */
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t index);
double   orc_uniform_at(uint64_t seed, uint64_t index);        /* in (0, 1] */
double   orc_normal_at(uint64_t seed, uint64_t index);         /* N(0,1) */
void     orc_fill_normal_f32(float* out, size_t n, uint64_t seed, double stddev);
void     orc_fill_normal_f16(uint16_t* out, size_t n, uint64_t seed, double stddev);
void     orc_fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed, double stddev);
/* GGUF blocks, nblocks * 34 (Q8_0) or * 18 (Q4_0) bytes.
 * Q8_0: qs uniform in [-127,127], d = f16(|N(0,wstd)| / 127).
 * Q4_0: codes uniform in [0,15],  d = f16(|N(0,wstd)| / 8). */
void     orc_fill_q8_0(uint8_t* blocks, size_t nblocks, uint64_t seed, double wstd);
void     orc_fill_q4_0(uint8_t* blocks, size_t nblocks, uint64_t seed, double wstd);

/* ---- GGUF block facts ---------------------------------------------------- */
#define ORC_QK 32
#define ORC_Q8_0_BLOCK_BYTES 34
#define ORC_Q4_0_BLOCK_BYTES 18
int    orc_ggml_type_size(int ggml_type);        /* bytes per block (F32 4, F16 2, Q4_0 18, Q8_0 34) */
int    orc_ggml_block_size(int ggml_type);       /* elements per block */
void   orc_dequant_q8_0(const uint8_t* blocks, float* out, size_t nblocks);
void   orc_dequant_q4_0(const uint8_t* blocks, float* out, size_t nblocks);

/* ---- restatements of gemm.cl (B is [K,N] row-major, fp16 bit patterns) ---- */
/* C16 receives the fp16 store, C32 (may be NULL) the fp32 accumulator. */
void orc_gemm_naive(const uint16_t* A, const uint16_t* B, uint16_t* C16, float* C32,
                    int M, int N, int K);
void orc_gemm_tiled(const uint16_t* A, const uint16_t* B, uint16_t* C16, float* C32,
                    int M, int N, int K);
void orc_gemm_image(const uint16_t* A, const uint16_t* B, uint16_t* C16, float* C32,
                    int M, int N, int K);
void orc_gemv(const uint16_t* x, const uint16_t* B, uint16_t* y16, float* y32, int N, int K);
/* the same on nthreads OpenMP threads (0: all); bit-identical results */
void orc_gemm_image_mt(const uint16_t* A, const uint16_t* B, uint16_t* C16, float* C32,
                       int M, int N, int K, int nthreads);
void orc_gemv_mt(const uint16_t* x, const uint16_t* B, uint16_t* y16, float* y32, int N, int K, int nthreads);

/* ---- the NT path: W is [N,K] (GGUF-native), y = X * W^T ---------------- */
/* fp32 fma chain over ascending k per output; OpenMP over rows when
 * nthreads > 1 (the result does not depend on the thread count). */
void orc_gemm_f32_nk(const float* X, const float* W, float* Y, int M, int N, int K, int nthreads);
void orc_gemm_f16_nk(const uint16_t* X, const uint16_t* W, float* Y, int M, int N, int K, int nthreads);
void orc_gemm_bf16_nk(const uint16_t* X, const uint16_t* W, float* Y, int M, int N, int K, int nthreads);
/* X fp32 [M,K]; W GGUF blocks, N rows of K/32 blocks. */
void orc_gemm_q8_0_nk(const float* X, const uint8_t* W, float* Y, int M, int N, int K, int nthreads);
void orc_gemm_q4_0_nk(const float* X, const uint8_t* W, float* Y, int M, int N, int K, int nthreads);
/* Batched NT GEMM with strides (in elements): C[b][m][n] = sum_k A[b][m][k] * B[b][n][k]. */
void orc_gemm_batched_f16(const uint16_t* A, const uint16_t* B, float* C, int batch,
                          int M, int N, int K, long lda, long ldb, long ldc,
                          long strideA, long strideB, long strideC);

/* ---- fp64 brute force: Y = X * W^T in fp64, S = sum |x*w| ---------------- */
void orc_gemm_f64_nk(const double* X, const double* W, double* Y, double* S,
                     int M, int N, int K, int nthreads);

/* ---- fused epilogue: Y[i] = act(Y[i] + bias[n]) * mul[i] + res[i] (fp64) -
 * act 0: none; 1: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
 * (src/kernels/activations.cl:68, the formula its comment states);
 * 2: x / (1 + exp(-x)) (activations.cl:22).  bias/mul/res may be NULL. */
double orc_gelu_tanh(double x);
double orc_silu(double x);
void orc_epilogue_f64(double* Y, const double* bias, const double* mul, const double* res, int act, int M, int N);

/* ---- attention (src/kernels/attention.cl:46-179 prefill, :197-295 decode) --
 * Q [seq_q][heads][D], K/V [seq_kv][heads][D] fp16 bits; per (query, head):
 * s_k = scale * sum_d Q[d] K[k][d] (fp64), keys with k > q + (seq_kv - seq_q)
 * masked when causal (attention.cl:96: kv_pos > query_pos when seq_q ==
 * seq_kv), p_k = exp(s_k - max) / sum, O[d] = sum_k p_k V[k][d].
 * Also returns A[q][h][d] = sum_k p_k |V[k][d]| (the error scale of O) and
 * R[q][h] = max_k scale * sum_d |Q[d] K[k][d]| (the error scale of a score). */
void orc_attention_f64(const uint16_t* Q, const uint16_t* K, const uint16_t* V, double* O, double* A, double* R,
                       int seq_q, int seq_kv, int heads, int D, int causal, double scale, int nthreads);

/* ---- LM-head token pick (src/models/moondream2.cpp:553-593) ---------------
 * orc_argmax_f16_reference: the reference's scan, literally: fp16 decode with
 * zero exponent -> 0 and all-ones exponent -> +-1e30, best = -1e30, strict '>'
 * from index 0.  orc_argmax: the same order for F32 (0), F16 (1) and BF16 (30)
 * rows with inf/NaN as +-inf; out[r] for each of `rows` rows of stride ld. */
int orc_argmax_f16_reference(const uint16_t* logits, int vocab);
void orc_argmax(const void* x, int dtype, int rows, int n, long ld, int* out);

int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
