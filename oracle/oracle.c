/*
 * oracle.c — CPU restatement of the MVLM matmul hot path (TEST INFRASTRUCTURE).
 * See oracle.h for what each function restates and how it is pinned.
 * Built with -ffp-contract=off so that only the explicit fmaf() calls fuse,
 * exactly as the reference's explicit fma() calls do.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* number formats                                                            */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary32 -> binary16, round to nearest even (the rounding vstore_half
 * uses by default, OpenCL C 6.15.6).  The reference's host-side converters
 * (benchmarks/gemm_bench.cpp:27-46) truncate and flush to zero; they are not
 * followed here. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                      /* inf / nan */
        if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);   /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                       /* below 2^-14: f16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;            /* <= 2^-25 -> 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                /* value / 2^-24 = m >> shift */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3FFu);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;   /* m * 2^-24, exact */
        return (sign ? -v : v);
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t orc_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t bias = 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)((x + bias) >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

void orc_f32_to_f16_array(const float* s, uint16_t* d, size_t n) { for (size_t i = 0; i < n; ++i) d[i] = orc_f32_to_f16(s[i]); }
void orc_f16_to_f32_array(const uint16_t* s, float* d, size_t n) { for (size_t i = 0; i < n; ++i) d[i] = orc_f16_to_f32(s[i]); }
void orc_f32_to_bf16_array(const float* s, uint16_t* d, size_t n) { for (size_t i = 0; i < n; ++i) d[i] = orc_f32_to_bf16(s[i]); }
void orc_bf16_to_f32_array(const uint16_t* s, float* d, size_t n) { for (size_t i = 0; i < n; ++i) d[i] = orc_bf16_to_f32(s[i]); }

/* ------------------------------------------------------------------------ */
/* seeded inputs                                                             */
/* ------------------------------------------------------------------------ */

/* SplitMix64 evaluated at counter `index` (state = seed + (index+1)*golden),
 * so any element can be produced independently (CPU or GPU). */
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1u) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

double orc_uniform_at(uint64_t seed, uint64_t index) {
    return (double)((orc_splitmix64_at(seed, index) >> 11) + 1u) * 0x1.0p-53;
}

/* Box-Muller on the pair (2j, 2j+1): even index -> r cos t, odd -> r sin t. */
double orc_normal_at(uint64_t seed, uint64_t index) {
    uint64_t j = index >> 1;
    double u1 = orc_uniform_at(seed, 2 * j);
    double u2 = orc_uniform_at(seed, 2 * j + 1);
    double r = sqrt(-2.0 * log(u1));
    double t = 6.283185307179586476925286766559 * u2;
    return (index & 1u) ? r * sin(t) : r * cos(t);
}

void orc_fill_normal_f32(float* out, size_t n, uint64_t seed, double sd) {
    for (size_t i = 0; i < n; ++i) out[i] = (float)(sd * orc_normal_at(seed, i));
}
void orc_fill_normal_f16(uint16_t* out, size_t n, uint64_t seed, double sd) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_f16((float)(sd * orc_normal_at(seed, i)));
}
void orc_fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed, double sd) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16((float)(sd * orc_normal_at(seed, i)));
}

/* Quant codes come from a second stream (seed ^ 0x5157) so scales and codes
 * are independent. */
#define ORC_CODE_STREAM 0x5157ull

void orc_fill_q8_0(uint8_t* blocks, size_t nblocks, uint64_t seed, double wstd) {
    for (size_t b = 0; b < nblocks; ++b) {
        uint8_t* blk = blocks + b * ORC_Q8_0_BLOCK_BYTES;
        uint16_t d = orc_f32_to_f16((float)(fabs(wstd * orc_normal_at(seed, b)) / 127.0));
        memcpy(blk, &d, 2);
        for (int j = 0; j < ORC_QK; ++j) {
            uint64_t r = orc_splitmix64_at(seed ^ ORC_CODE_STREAM, (uint64_t)b * ORC_QK + (uint64_t)j);
            int q = (int)(r % 255u) - 127;
            blk[2 + j] = (uint8_t)(int8_t)q;
        }
    }
}

void orc_fill_q4_0(uint8_t* blocks, size_t nblocks, uint64_t seed, double wstd) {
    for (size_t b = 0; b < nblocks; ++b) {
        uint8_t* blk = blocks + b * ORC_Q4_0_BLOCK_BYTES;
        uint16_t d = orc_f32_to_f16((float)(fabs(wstd * orc_normal_at(seed, b)) / 8.0));
        memcpy(blk, &d, 2);
        uint8_t code[ORC_QK];
        for (int j = 0; j < ORC_QK; ++j)
            code[j] = (uint8_t)(orc_splitmix64_at(seed ^ ORC_CODE_STREAM, (uint64_t)b * ORC_QK + (uint64_t)j) & 15u);
        for (int j = 0; j < ORC_QK / 2; ++j) blk[2 + j] = (uint8_t)(code[j] | (code[j + 16] << 4));
    }
}

/* ------------------------------------------------------------------------ */
/* GGUF block facts (ggml type ids as in src/models/gguf_loader.h:12-31)      */
/* ------------------------------------------------------------------------ */

int orc_ggml_type_size(int t) {
    switch (t) {
        case 0: return 4;    /* F32 */
        case 1: return 2;    /* F16 */
        case 2: return 18;   /* Q4_0: fp16 d + 16 bytes of nibbles */
        case 8: return 34;   /* Q8_0: fp16 d + 32 int8 */
        case 30: return 2;   /* BF16 */
        default: return 0;
    }
}

int orc_ggml_block_size(int t) {
    switch (t) {
        case 0: case 1: case 30: return 1;
        case 2: case 8: return 32;
        default: return 0;
    }
}

/* Q8_0: w_j = d * qs_j (fp16 d widened exactly, product exact in fp32). */
void orc_dequant_q8_0(const uint8_t* blocks, float* out, size_t nblocks) {
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* blk = blocks + b * ORC_Q8_0_BLOCK_BYTES;
        uint16_t dh; memcpy(&dh, blk, 2);
        float d = orc_f16_to_f32(dh);
        for (int j = 0; j < ORC_QK; ++j) out[b * ORC_QK + j] = (float)(int8_t)blk[2 + j] * d;
    }
}

/* Q4_0: w_j = ((qs_j & 15) - 8) * d and w_{j+16} = ((qs_j >> 4) - 8) * d, j < 16. */
void orc_dequant_q4_0(const uint8_t* blocks, float* out, size_t nblocks) {
    for (size_t b = 0; b < nblocks; ++b) {
        const uint8_t* blk = blocks + b * ORC_Q4_0_BLOCK_BYTES;
        uint16_t dh; memcpy(&dh, blk, 2);
        float d = orc_f16_to_f32(dh);
        for (int j = 0; j < ORC_QK / 2; ++j) {
            out[b * ORC_QK + j]      = (float)((int)(blk[2 + j] & 15) - 8) * d;
            out[b * ORC_QK + j + 16] = (float)((int)(blk[2 + j] >> 4) - 8) * d;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* restatements of src/kernels/gemm.cl                                       */
/* ------------------------------------------------------------------------ */

#define H2F orc_f16_to_f32

/* gemm.cl:26-51: one work-item per (row, col); acc = fma(A[row,k], B[k,col], acc)
 * for k = 0..K-1; vstore_half(acc). */
void orc_gemm_naive(const uint16_t* A, const uint16_t* B, uint16_t* C16, float* C32,
                    int M, int N, int K) {
    for (int row = 0; row < M; ++row)
        for (int col = 0; col < N; ++col) {
            float acc = 0.0f;
            for (int k = 0; k < K; ++k)
                acc = fmaf(H2F(A[(size_t)row * K + k]), H2F(B[(size_t)k * N + col]), acc);
            if (C16) C16[(size_t)row * N + col] = orc_f32_to_f16(acc);
            if (C32) C32[(size_t)row * N + col] = acc;
        }
}

/* gemm.cl:64-136 with TILE_M = TILE_N = TILE_K = 8: work-groups of 8x8, the
 * K loop walks 8-wide tiles staged in local memory (zero outside the matrix),
 * and each item accumulates its 8 products per tile in ascending k. */
void orc_gemm_tiled(const uint16_t* A, const uint16_t* B, uint16_t* C16, float* C32,
                    int M, int N, int K) {
    enum { T = 8 };
    int ntiles = (K + T - 1) / T;
    int groups_m = (M + T - 1) / T, groups_n = (N + T - 1) / T;
    float* acc = (float*)malloc(sizeof(float) * T * T);
    for (int gm = 0; gm < groups_m; ++gm)
        for (int gn = 0; gn < groups_n; ++gn) {
            for (int i = 0; i < T * T; ++i) acc[i] = 0.0f;
            for (int t = 0; t < ntiles; ++t) {
                uint16_t tA[T][T], tB[T][T];
                for (int lr = 0; lr < T; ++lr)
                    for (int lc = 0; lc < T; ++lc) {
                        int grow = gm * T + lr, gcol = gn * T + lc;
                        int a_col = t * T + lc, b_row = t * T + lr;
                        tA[lr][lc] = (grow < M && a_col < K) ? A[(size_t)grow * K + a_col] : 0;
                        tB[lr][lc] = (b_row < K && gcol < N) ? B[(size_t)b_row * N + gcol] : 0;
                    }
                for (int lr = 0; lr < T; ++lr)
                    for (int lc = 0; lc < T; ++lc)
                        for (int k = 0; k < T; ++k)
                            acc[lr * T + lc] = fmaf(H2F(tA[lr][k]), H2F(tB[k][lc]), acc[lr * T + lc]);
            }
            for (int lr = 0; lr < T; ++lr)
                for (int lc = 0; lc < T; ++lc) {
                    int grow = gm * T + lr, gcol = gn * T + lc;
                    if (grow < M && gcol < N) {
                        if (C16) C16[(size_t)grow * N + gcol] = orc_f32_to_f16(acc[lr * T + lc]);
                        if (C32) C32[(size_t)grow * N + gcol] = acc[lr * T + lc];
                    }
                }
        }
    free(acc);
}

/* memory.cpp:28-79 packs B[K,N] into an RGBA-half image of width ceil(N/4),
 * height K, zero-padding the columns to a multiple of 4; gemm.cl:157-200 then
 * lets each item produce 4 adjacent columns (float4 fma over ascending k) and
 * stores min(4, N - col_base) of them. */
void orc_gemm_image_mt(const uint16_t* A, const uint16_t* B, uint16_t* C16, float* C32,
                       int M, int N, int K, int nthreads) {
    int width = (N + 3) / 4, padded = width * 4;
    int nt = nthreads > 0 ? nthreads : orc_max_threads();
    uint16_t* img = (uint16_t*)calloc((size_t)K * padded, sizeof(uint16_t));
    for (int k = 0; k < K; ++k) memcpy(img + (size_t)k * padded, B + (size_t)k * N, sizeof(uint16_t) * N);
    /* rows are independent work items: threads change nothing in the results */
    #pragma omp parallel for schedule(static) num_threads(nt)
    for (int row = 0; row < M; ++row)
        for (int col4 = 0; col4 < width; ++col4) {
            int col_base = col4 * 4;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int k = 0; k < K; ++k) {
                float a = H2F(A[(size_t)row * K + k]);
                const uint16_t* t = img + (size_t)k * padded + col_base;
                for (int c = 0; c < 4; ++c) acc[c] = fmaf(a, H2F(t[c]), acc[c]);
            }
            int remaining = N - col_base;
            for (int c = 0; c < 4 && c < remaining; ++c) {
                if (C16) C16[(size_t)row * N + col_base + c] = orc_f32_to_f16(acc[c]);
                if (C32) C32[(size_t)row * N + col_base + c] = acc[c];
            }
        }
    free(img);
}

void orc_gemm_image(const uint16_t* A, const uint16_t* B, uint16_t* C16, float* C32, int M, int N, int K) {
    orc_gemm_image_mt(A, B, C16, C32, M, N, K, 1);
}

/* gemm.cl:215-270 as launched by compute.cpp:141-147: one 256-item group per
 * image column (4 outputs); item lid accumulates k = lid, lid+256, ... with a
 * float4 fma; then scratch[lid] += scratch[lid+stride] for stride = 128..1. */
void orc_gemv_mt(const uint16_t* x, const uint16_t* B, uint16_t* y16, float* y32, int N, int K, int nthreads) {
    enum { WG = 256 };
    int width = (N + 3) / 4;
    int nt = nthreads > 0 ? nthreads : orc_max_threads();
    /* work-groups (4 outputs each) are independent: threads change nothing */
    #pragma omp parallel for schedule(static) num_threads(nt)
    for (int col4 = 0; col4 < width; ++col4) {
        float scratch[WG][4];
        int col_base = col4 * 4;
        for (int lid = 0; lid < WG; ++lid) {
            float p[4] = {0.f, 0.f, 0.f, 0.f};
            for (int k = lid; k < K; k += WG) {
                float xv = H2F(x[k]);
                for (int c = 0; c < 4; ++c) {
                    int col = col_base + c;
                    float w = (col < N) ? H2F(B[(size_t)k * N + col]) : 0.0f;  /* zero pad */
                    p[c] = fmaf(xv, w, p[c]);
                }
            }
            for (int c = 0; c < 4; ++c) scratch[lid][c] = p[c];
        }
        for (int stride = WG >> 1; stride > 0; stride >>= 1)
            for (int lid = 0; lid < stride; ++lid)
                for (int c = 0; c < 4; ++c) scratch[lid][c] = scratch[lid][c] + scratch[lid + stride][c];
        int remaining = N - col_base;
        for (int c = 0; c < 4 && c < remaining; ++c) {
            if (y16) y16[col_base + c] = orc_f32_to_f16(scratch[0][c]);
            if (y32) y32[col_base + c] = scratch[0][c];
        }
    }
}

void orc_gemv(const uint16_t* x, const uint16_t* B, uint16_t* y16, float* y32, int N, int K) {
    orc_gemv_mt(x, B, y16, y32, N, K, 1);
}

/* ------------------------------------------------------------------------ */
/* the NT path (weights [N,K]), fp32 fma chain in ascending k                 */
/* ------------------------------------------------------------------------ */

static int clamp_threads(int n) {
#ifdef _OPENMP
    if (n <= 0) n = omp_get_max_threads();
    return n;
#else
    (void)n;
    return 1;
#endif
}

int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Rows are processed 8 at a time with a [k][r] staging tile so the compiler
 * can vectorise across the 8 independent fma chains; each chain is still the
 * ascending-k sequence of one output, so the result equals the scalar loop.
 * `load` writes the exact fp32 values of W[n, k0 .. k0+kn) into dst. */
#define ROWS 8
typedef void (*row_loader)(const void* W, int n, int k0, int kn, int K, float* dst);

static void nt_gemm(const float* X, const void* W, row_loader load, float* Y,
                    int M, int N, int K, int nthreads) {
    int nt = clamp_threads(nthreads);
    int nrb = (N + ROWS - 1) / ROWS;
    #pragma omp parallel for schedule(static) num_threads(nt)
    for (int rb = 0; rb < nrb; ++rb) {
        float wt[ORC_QK][ROWS];
        float seg[ORC_QK];
        int n0 = rb * ROWS;
        int nr = (N - n0 < ROWS) ? N - n0 : ROWS;
        for (int m = 0; m < M; ++m) {
            float acc[ROWS];
            for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
            for (int k0 = 0; k0 < K; k0 += ORC_QK) {
                int kn = (K - k0 < ORC_QK) ? K - k0 : ORC_QK;
                for (int j = 0; j < ORC_QK; ++j)
                    for (int r = 0; r < ROWS; ++r) wt[j][r] = 0.0f;
                for (int r = 0; r < nr; ++r) {
                    load(W, n0 + r, k0, kn, K, seg);
                    for (int j = 0; j < kn; ++j) wt[j][r] = seg[j];
                }
                const float* xr = X + (size_t)m * K + k0;
                for (int j = 0; j < kn; ++j) {
                    float xv = xr[j];
                    for (int r = 0; r < ROWS; ++r) acc[r] = fmaf(xv, wt[j][r], acc[r]);
                }
            }
            for (int r = 0; r < nr; ++r) Y[(size_t)m * N + n0 + r] = acc[r];
        }
    }
}

static void load_f32(const void* W, int n, int k0, int kn, int K, float* dst) {
    const float* w = (const float*)W + (size_t)n * K + k0;
    for (int j = 0; j < kn; ++j) dst[j] = w[j];
}
static void load_f16(const void* W, int n, int k0, int kn, int K, float* dst) {
    const uint16_t* w = (const uint16_t*)W + (size_t)n * K + k0;
    for (int j = 0; j < kn; ++j) dst[j] = orc_f16_to_f32(w[j]);
}
static void load_bf16(const void* W, int n, int k0, int kn, int K, float* dst) {
    const uint16_t* w = (const uint16_t*)W + (size_t)n * K + k0;
    for (int j = 0; j < kn; ++j) dst[j] = orc_bf16_to_f32(w[j]);
}
/* quantized rows: K is a multiple of 32 and k0 a block boundary */
static void load_q8_0(const void* W, int n, int k0, int kn, int K, float* dst) {
    (void)kn;
    const uint8_t* blk = (const uint8_t*)W + ((size_t)n * (K / ORC_QK) + (size_t)(k0 / ORC_QK)) * ORC_Q8_0_BLOCK_BYTES;
    orc_dequant_q8_0(blk, dst, 1);
}
static void load_q4_0(const void* W, int n, int k0, int kn, int K, float* dst) {
    (void)kn;
    const uint8_t* blk = (const uint8_t*)W + ((size_t)n * (K / ORC_QK) + (size_t)(k0 / ORC_QK)) * ORC_Q4_0_BLOCK_BYTES;
    orc_dequant_q4_0(blk, dst, 1);
}

static float* widen(const uint16_t* X, size_t n, float (*cvt)(uint16_t)) {
    float* out = (float*)malloc(sizeof(float) * (n ? n : 1));
    for (size_t i = 0; i < n; ++i) out[i] = cvt(X[i]);
    return out;
}

void orc_gemm_f32_nk(const float* X, const float* W, float* Y, int M, int N, int K, int nthreads) {
    nt_gemm(X, W, load_f32, Y, M, N, K, nthreads);
}
void orc_gemm_f16_nk(const uint16_t* X, const uint16_t* W, float* Y, int M, int N, int K, int nthreads) {
    float* Xf = widen(X, (size_t)M * K, orc_f16_to_f32);
    nt_gemm(Xf, W, load_f16, Y, M, N, K, nthreads);
    free(Xf);
}
void orc_gemm_bf16_nk(const uint16_t* X, const uint16_t* W, float* Y, int M, int N, int K, int nthreads) {
    float* Xf = widen(X, (size_t)M * K, orc_bf16_to_f32);
    nt_gemm(Xf, W, load_bf16, Y, M, N, K, nthreads);
    free(Xf);
}
void orc_gemm_q8_0_nk(const float* X, const uint8_t* W, float* Y, int M, int N, int K, int nthreads) {
    nt_gemm(X, W, load_q8_0, Y, M, N, K, nthreads);
}
void orc_gemm_q4_0_nk(const float* X, const uint8_t* W, float* Y, int M, int N, int K, int nthreads) {
    nt_gemm(X, W, load_q4_0, Y, M, N, K, nthreads);
}

void orc_gemm_batched_f16(const uint16_t* A, const uint16_t* B, float* C, int batch,
                          int M, int N, int K, long lda, long ldb, long ldc,
                          long strideA, long strideB, long strideC) {
    for (int b = 0; b < batch; ++b) {
        const uint16_t* Ab = A + (size_t)b * strideA;
        const uint16_t* Bb = B + (size_t)b * strideB;
        float* Cb = C + (size_t)b * strideC;
        #pragma omp parallel for schedule(static)
        for (int m = 0; m < M; ++m)
            for (int n = 0; n < N; ++n) {
                float acc = 0.0f;
                for (int k = 0; k < K; ++k)
                    acc = fmaf(H2F(Ab[(size_t)m * lda + k]), H2F(Bb[(size_t)n * ldb + k]), acc);
                Cb[(size_t)m * ldc + n] = acc;
            }
    }
}

void orc_gemm_f64_nk(const double* X, const double* W, double* Y, double* S,
                     int M, int N, int K, int nthreads) {
    int nt = clamp_threads(nthreads);
    #pragma omp parallel for schedule(static) num_threads(nt)
    for (int n = 0; n < N; ++n)
        for (int m = 0; m < M; ++m) {
            double acc = 0.0, s = 0.0;
            for (int k = 0; k < K; ++k) {
                double p = X[(size_t)m * K + k] * W[(size_t)n * K + k];
                acc += p;
                s += fabs(p);
            }
            Y[(size_t)m * N + n] = acc;
            if (S) S[(size_t)m * N + n] = s;
        }
}

/* ---- fused epilogue -------------------------------------------------------
 * activations.cl:66-118 (gelu), :22-60 (silu), vision.cl:178-186 / 433-436
 * (bias), activations.cl:259-290 (vector_add residual), :204-255 (gate). */
double orc_gelu_tanh(double x) {
    const double c = sqrt(2.0 / 3.14159265358979323846);
    return 0.5 * x * (1.0 + tanh(c * (x + 0.044715 * x * x * x)));
}

double orc_silu(double x) { return x / (1.0 + exp(-x)); }

void orc_epilogue_f64(double* Y, const double* bias, const double* mul, const double* res, int act, int M, int N) {
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            const size_t i = (size_t)m * N + n;
            double v = Y[i];
            if (bias) v += bias[n];
            if (act == 1) v = orc_gelu_tanh(v);
            else if (act == 2) v = orc_silu(v);
            if (mul) v *= mul[i];
            if (res) v += res[i];
            Y[i] = v;
        }
}

void orc_attention_f64(const uint16_t* Q, const uint16_t* K, const uint16_t* V, double* O, double* A, double* R,
                       int seq_q, int seq_kv, int heads, int D, int causal, double scale, int nthreads) {
    const int nt = clamp_threads(nthreads);
    const size_t row = (size_t)heads * D;
    const int shift = seq_kv - seq_q;
    #pragma omp parallel num_threads(nt)
    {
        double* s = (double*)malloc(sizeof(double) * (size_t)(seq_kv > 0 ? seq_kv : 1));
        double* q = (double*)malloc(sizeof(double) * (size_t)D);
        #pragma omp for schedule(dynamic, 4)
        for (long qh = 0; qh < (long)seq_q * heads; ++qh) {
            const int qi = (int)(qh / heads), h = (int)(qh % heads);
            const uint16_t* qp = Q + (size_t)qi * row + (size_t)h * D;
            for (int d = 0; d < D; ++d) q[d] = H2F(qp[d]);
            int last = seq_kv - 1;
            if (causal && qi + shift < last) last = qi + shift;
            double m = -INFINITY, r = 0.0;
            for (int k = 0; k <= last; ++k) {
                const uint16_t* kp = K + (size_t)k * row + (size_t)h * D;
                double acc = 0.0, mag = 0.0;
                for (int d = 0; d < D; ++d) {
                    const double pr = q[d] * H2F(kp[d]);
                    acc += pr;
                    mag += fabs(pr);
                }
                s[k] = scale * acc;
                if (s[k] > m) m = s[k];
                if (scale * mag > r) r = scale * mag;
            }
            double l = 0.0;
            for (int k = 0; k <= last; ++k) {
                s[k] = exp(s[k] - m);
                l += s[k];
            }
            double* o = O + (size_t)qi * row + (size_t)h * D;
            double* a = A + (size_t)qi * row + (size_t)h * D;
            for (int d = 0; d < D; ++d) o[d] = a[d] = 0.0;
            for (int k = 0; k <= last; ++k) {
                const uint16_t* vp = V + (size_t)k * row + (size_t)h * D;
                const double w = s[k] / l;
                for (int d = 0; d < D; ++d) {
                    const double v = H2F(vp[d]);
                    o[d] += w * v;
                    a[d] += w * fabs(v);
                }
            }
            R[qh] = r;
        }
        free(s);
        free(q);
    }
}

int orc_argmax_f16_reference(const uint16_t* logits, int vocab) {
    int best_id = 0;
    float best_val = -1e30f;
    for (int i = 0; i < vocab; i++) {
        const uint16_t h = logits[i];
        const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
        const uint32_t e = (h >> 10) & 0x1F, mant = h & 0x3FF;
        float val;
        if (e == 0) {
            val = 0.0f;
        } else if (e == 31) {
            val = (sign ? -1.0f : 1.0f) * 1e30f;
        } else {
            const uint32_t f32 = sign | ((e - 15 + 127) << 23) | (mant << 13);
            memcpy(&val, &f32, 4);
        }
        if (val > best_val) {
            best_val = val;
            best_id = i;
        }
    }
    return best_id;
}

static float argmax_key(const void* row, long i, int dtype) {
    if (dtype == 0) {
        uint32_t b;
        memcpy(&b, (const uint8_t*)row + 4 * i, 4);
        const uint32_t e = (b >> 23) & 0xFF;
        if (e == 0xFF) return (b >> 31) ? -INFINITY : INFINITY;
        if (e == 0) return 0.0f;
        float v;
        memcpy(&v, &b, 4);
        return v;
    }
    const uint16_t h = ((const uint16_t*)row)[i];
    if (dtype == 1) {
        const uint32_t e = (h >> 10) & 0x1F;
        if (e == 0x1F) return (h >> 15) ? -INFINITY : INFINITY;
        return e == 0 ? 0.0f : orc_f16_to_f32(h);
    }
    const uint32_t e = (h >> 7) & 0xFF;
    if (e == 0xFF) return (h >> 15) ? -INFINITY : INFINITY;
    return e == 0 ? 0.0f : orc_bf16_to_f32(h);
}

void orc_argmax(const void* x, int dtype, int rows, int n, long ld, int* out) {
    const size_t es = dtype == 0 ? 4 : 2;
    for (int r = 0; r < rows; ++r) {
        const void* row = (const uint8_t*)x + (size_t)r * ld * es;
        int best = 0;
        float bk = argmax_key(row, 0, dtype);
        for (int i = 1; i < n; ++i) {
            const float k = argmax_key(row, i, dtype);
            if (k > bk) {
                bk = k;
                best = i;
            }
        }
        out[r] = best;
    }
}
