// Launch entry points and plans.
//
// Every launch is first turned into a validated Op (all checks on the host,
// before anything is enqueued), then enqueued by enqueue_op.  The direct
// entry points (mvlm_gemm_*, mvlm_gemv*) do both at once, matching the
// reference dispatchers (src/engine/compute.cpp:28-152); a plan validates at
// add time and enqueues from native code on every run, eagerly or by
// replaying a captured HIP graph.
#include "common.h"

#include <cmath>
#include <new>
#include <vector>

using namespace mvlm;

namespace {

enum OpKind { OP_GEMM_NAIVE, OP_GEMM_TILED, OP_GEMV_EXACT, OP_GEMM_MFMA, OP_GEMV_DENSE, OP_GEMV_QUANT, OP_GEMV_GROUP, OP_ATTENTION,
              OP_ATTN_STEP, OP_ARGMAX };

struct Op {
    OpKind kind;
    const void* a = nullptr;      // A / x / X
    const void* b = nullptr;      // B (naive, tiled, batched); K (attention)
    const void* v = nullptr;      // V (attention)
    void* c = nullptr;            // C / y / Y
    const mvlm_weight* w = nullptr;
    int a_dtype = MVLM_F16, c_dtype = MVLM_F32;
    int batch = 1, M = 0, N = 0, K = 0;
    int64_t lda = 0, ldb = 0, ldc = 0, sA = 0, sB = 0, sC = 0;
    int kread_b = 0;              // B rows readable (zero padded) up to this K
    int num_cus = 256;
    // grouped GEMV
    int gcount = 0;
    const void* gx[MVLM_MAX_GROUP] = {};
    const mvlm_weight* gw[MVLM_MAX_GROUP] = {};
    void* gy[MVLM_MAX_GROUP] = {};
    int gyd[MVLM_MAX_GROUP] = {};
    Epilogue gep[MVLM_MAX_GROUP]; // per-entry epilogues of a grouped launch
    Epilogue ep;                  // fused epilogue (GEMM MFMA, GEMV)
    // attention: M = seq_q, N = seq_kv, batch = heads, K = head_dim
    int causal = 0;
    float scale = 0.0f;
    void* workspace = nullptr;    // attention key splits, GEMM K splits
    size_t workspace_bytes = 0;
    // plan fusion: a grouped GEMV whose launch can also compute a decode
    // attention entry next to it; 1: the entry before it (some entries read
    // its output as x), 2: the entry after it (a decode step whose q, k, v
    // one entry writes)
    int attn_carry = 0;
    StreamAttnDesc attn;
};

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return a && b && an && bn && x < y + bn && y < x + an;
}

int need(const mvlm_buffer* b, size_t bytes, const char* fn, const char* name) {
    if (b->bytes < bytes)
        return set_error(MVLM_ERR_BUFFER_TOO_SMALL, "%s: %s holds %zu bytes, %zu needed", fn, name, b->bytes, bytes);
    return MVLM_OK;
}

#define NEED(buf, bytes, name)                                   \
    do {                                                         \
        int _st = need((buf), (bytes), fn, (name));              \
        if (_st != MVLM_OK) return _st;                          \
    } while (0)

// Validates a caller's epilogue for an [M][N] output of dtype c_dtype.
int make_epilogue(mvlm_device* dev, const mvlm_epilogue* in, int M, int N, int c_dtype, const char* fn,
                  Epilogue* out) {
    *out = Epilogue{};
    if (!in) return MVLM_OK;
    REQUIRE(in->activation >= MVLM_ACT_NONE && in->activation <= MVLM_ACT_SILU, "%s: unknown activation %d", fn,
            in->activation);
    const size_t es = dtype_size(c_dtype);
    if (in->bias) {
        REQUIRE(in->bias->dev == dev, "%s: bias belongs to another device", fn);
        NEED(in->bias, (size_t)N * es, "bias");
        REQUIRE((uintptr_t)in->bias->ptr % es == 0, "%s: bias does not start at a multiple of %zu bytes", fn, es);
        out->bias = in->bias->ptr;
    }
    if (in->mul) {
        REQUIRE(in->mul->dev == dev, "%s: mul belongs to another device", fn);
        NEED(in->mul, (size_t)M * N * es, "mul");
        REQUIRE((uintptr_t)in->mul->ptr % es == 0, "%s: mul does not start at a multiple of %zu bytes", fn, es);
        out->mul = in->mul->ptr;
    }
    if (in->residual) {
        REQUIRE(in->residual->dev == dev, "%s: residual belongs to another device", fn);
        NEED(in->residual, (size_t)M * N * es, "residual");
        REQUIRE((uintptr_t)in->residual->ptr % es == 0, "%s: residual does not start at a multiple of %zu bytes", fn, es);
        out->res = in->residual->ptr;
    }
    out->act = in->activation;
    out->dtype = c_dtype;
    return MVLM_OK;
}

int make_ref_gemm(OpKind kind, mvlm_device* dev, const mvlm_buffer* A, const mvlm_buffer* B, mvlm_buffer* C,
                  int M, int N, int K, const char* fn, Op* op) {
    REQUIRE(dev && A && B && C, "%s: null argument", fn);
    REQUIRE(A->dev == dev && B->dev == dev && C->dev == dev, "%s: buffers belong to another device", fn);
    REQUIRE(M > 0 && N > 0 && K > 0, "%s: M=%d N=%d K=%d must be positive", fn, M, N, K);
    NEED(A, (size_t)M * K * 2, "A");
    NEED(B, (size_t)K * N * 2, "B");
    NEED(C, (size_t)M * N * 2, "C");
    op->kind = kind;
    op->a = A->ptr; op->b = B->ptr; op->c = C->ptr;
    op->M = M; op->N = N; op->K = K;
    return MVLM_OK;
}

int make_gemv_exact(mvlm_device* dev, const mvlm_buffer* x, const mvlm_weight* W, mvlm_buffer* y, int N, int K,
                    const char* fn, Op* op) {
    REQUIRE(dev && x && W && y, "%s: null argument", fn);
    REQUIRE(x->dev == dev && W->dev == dev && y->dev == dev, "%s: handles belong to another device", fn);
    REQUIRE(N > 0 && K > 0, "%s: N=%d K=%d must be positive", fn, N, K);
    REQUIRE(W->N == N && W->K == K, "%s: weight is [%d x %d], call asks for N=%d K=%d", fn, W->N, W->K, N, K);
    REQUIRE(W->dtype == MVLM_F16, "%s: weight dtype %d is not F16", fn, W->dtype);
    REQUIRE(((uintptr_t)x->ptr & 7u) == 0, "%s: x must be 8-byte aligned", fn);
    NEED(x, (size_t)K * 2, "x");
    NEED(y, (size_t)N * 2, "y");
    op->kind = OP_GEMV_EXACT;
    op->a = x->ptr; op->w = W; op->c = y->ptr;
    op->M = 1; op->N = N; op->K = K;
    return MVLM_OK;
}

// The op of a packed-weight GEMM, all but its workspace (op->workspace_bytes
// says how much it needs).
int make_gemm_packed_op(mvlm_device* dev, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W, mvlm_buffer* C,
                        int c_dtype, int M, int N, int K, const char* fn, Op* op) {
    REQUIRE(dev && A && W && C, "%s: null argument", fn);
    REQUIRE(A->dev == dev && W->dev == dev && C->dev == dev, "%s: handles belong to another device", fn);
    REQUIRE(M > 0 && N > 0 && K > 0, "%s: M=%d N=%d K=%d must be positive", fn, M, N, K);
    REQUIRE(W->N == N && W->K == K, "%s: weight is [%d x %d], call asks for N=%d K=%d", fn, W->N, W->K, N, K);
    REQUIRE(W->dtype == MVLM_F16 || W->dtype == MVLM_BF16, "%s: weight dtype %d is not F16/BF16", fn, W->dtype);
    REQUIRE(a_dtype == W->dtype, "%s: activation dtype %d differs from weight dtype %d", fn, a_dtype, W->dtype);
    REQUIRE(is_dense(c_dtype), "%s: output dtype %d is not F32/F16/BF16", fn, c_dtype);
    REQUIRE(aligned16(A->ptr) && aligned16(C->ptr), "%s: A and C must be 16-byte aligned", fn);
    NEED(A, (size_t)M * K * 2, "A");
    NEED(C, (size_t)M * N * dtype_size(c_dtype), "C");
    op->kind = OP_GEMM_MFMA;
    op->a = A->ptr; op->b = W->data; op->c = C->ptr; op->w = W;
    op->a_dtype = a_dtype; op->c_dtype = c_dtype;
    op->M = M; op->N = N; op->K = K;
    op->lda = K; op->ldb = W->ld; op->ldc = N;
    op->kread_b = (int)W->ld;     // packed rows are zero padded to ld = roundup(K, 64)
    op->num_cus = dev->prop.multiProcessorCount;
    op->workspace_bytes = gemm_workspace_bytes(1, M, N, K, op->lda, op->ldb, 0, 0, op->kread_b, op->num_cus);
    return MVLM_OK;
}

int make_gemm_packed(mvlm_device* dev, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W, mvlm_buffer* C,
                     int c_dtype, int M, int N, int K, const char* fn, Op* op) {
    const int st = make_gemm_packed_op(dev, A, a_dtype, W, C, c_dtype, M, N, K, fn, op);
    return st != MVLM_OK ? st : device_scratch(dev, op->workspace_bytes, &op->workspace);
}

int make_gemm_batched(mvlm_device* dev, const mvlm_buffer* A, const mvlm_buffer* B, mvlm_buffer* C, int batch,
                      int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc, int64_t sA, int64_t sB,
                      int64_t sC, const char* fn, Op* op) {
    REQUIRE(dev && A && B && C, "%s: null argument", fn);
    REQUIRE(A->dev == dev && B->dev == dev && C->dev == dev, "%s: buffers belong to another device", fn);
    REQUIRE(batch > 0 && M > 0 && N > 0 && K > 0, "%s: batch=%d M=%d N=%d K=%d must be positive", fn, batch, M, N, K);
    REQUIRE(lda >= K && ldb >= K && ldc >= N, "%s: leading dimensions too small", fn);
    REQUIRE(sA >= 0 && sB >= 0 && sC >= 0, "%s: negative batch stride", fn);
    REQUIRE(aligned16(A->ptr) && aligned16(B->ptr) && ((uintptr_t)C->ptr & 3u) == 0,
            "%s: A and B must be 16-byte aligned, C 4-byte aligned", fn);
    NEED(A, ((size_t)(batch - 1) * sA + (size_t)(M - 1) * lda + K) * 2, "A");
    NEED(B, ((size_t)(batch - 1) * sB + (size_t)(N - 1) * ldb + K) * 2, "B");
    NEED(C, ((size_t)(batch - 1) * sC + (size_t)(M - 1) * ldc + N) * 4, "C");
    op->kind = OP_GEMM_MFMA;
    op->a = A->ptr; op->b = B->ptr; op->c = C->ptr;
    op->a_dtype = MVLM_F16; op->c_dtype = MVLM_F32;
    op->batch = batch; op->M = M; op->N = N; op->K = K;
    op->lda = lda; op->ldb = ldb; op->ldc = ldc; op->sA = sA; op->sB = sB; op->sC = sC;
    op->kread_b = K;
    op->num_cus = dev->prop.multiProcessorCount;
    op->workspace_bytes = gemm_workspace_bytes(batch, M, N, K, lda, ldb, sA, sB, K, op->num_cus);
    return device_scratch(dev, op->workspace_bytes, &op->workspace);
}

int make_attention(mvlm_device* dev, const mvlm_buffer* Q, const mvlm_buffer* K, const mvlm_buffer* V,
                   mvlm_buffer* O, int o_dtype, int seq_q, int seq_kv, int heads, int head_dim, int causal,
                   float scale, const char* fn, Op* op) {
    REQUIRE(dev && Q && K && V && O, "%s: null argument", fn);
    REQUIRE(Q->dev == dev && K->dev == dev && V->dev == dev && O->dev == dev, "%s: buffers belong to another device",
            fn);
    REQUIRE(seq_q > 0 && seq_kv > 0 && heads > 0 && head_dim > 0,
            "%s: seq_q=%d seq_kv=%d num_heads=%d head_dim=%d must be positive", fn, seq_q, seq_kv, heads, head_dim);
    REQUIRE(o_dtype == MVLM_F16 || o_dtype == MVLM_F32, "%s: output dtype %d is not F16/F32", fn, o_dtype);
    REQUIRE(!causal || seq_q <= seq_kv, "%s: causal attention needs seq_q (%d) <= seq_kv (%d)", fn, seq_q, seq_kv);
    REQUIRE(scale >= 0.0f && scale < INFINITY, "%s: scale %g must be finite and non-negative", fn, (double)scale);
    if (head_dim % 8 != 0 || head_dim > 128)
        return set_error(MVLM_ERR_UNSUPPORTED, "%s: head_dim=%d must be a multiple of 8 and at most 128", fn,
                         head_dim);
    REQUIRE(heads <= 65535 && (int64_t)heads * head_dim <= (1 << 24) && (int64_t)seq_q * heads <= (1 << 30) &&
                (int64_t)seq_kv * heads <= (1 << 30),
            "%s: shape too large", fn);
    REQUIRE(aligned16(Q->ptr) && aligned16(K->ptr) && aligned16(V->ptr) && aligned16(O->ptr),
            "%s: Q, K, V and O must be 16-byte aligned", fn);
    const size_t row = (size_t)heads * head_dim;
    // the kernel addresses Q, K and V with 32-bit buffer offsets (keys read up
    // to 576 positions past the end return zeros)
    if ((size_t)seq_q * row * 2 > (1u << 30) || ((size_t)seq_kv + 576) * row * 2 > (1u << 30))
        return set_error(MVLM_ERR_UNSUPPORTED, "%s: Q, K or V larger than 1 GiB", fn);
    NEED(Q, (size_t)seq_q * row * 2, "Q");
    NEED(K, (size_t)seq_kv * row * 2, "K");
    NEED(V, (size_t)seq_kv * row * 2, "V");
    NEED(O, (size_t)seq_q * row * dtype_size(o_dtype), "O");
    op->kind = OP_ATTENTION;
    op->a = Q->ptr; op->b = K->ptr; op->v = V->ptr; op->c = O->ptr;
    op->c_dtype = o_dtype;
    op->M = seq_q; op->N = seq_kv; op->batch = heads; op->K = head_dim;
    op->causal = causal ? 1 : 0;
    op->scale = scale == 0.0f ? 1.0f / sqrtf((float)head_dim) : scale;
    op->num_cus = dev->prop.multiProcessorCount;
    op->workspace_bytes = attention_workspace_bytes(seq_q, seq_kv, heads, head_dim, op->num_cus);
    return device_scratch(dev, op->workspace_bytes, &op->workspace);
}

// Decode attention step (mode 1 of StreamAttnDesc): qkv fp32 [3][heads][D],
// caches fp16 [cached + 1][heads][D] (row `cached` written), O fp32 [heads][D].
int make_attn_step(mvlm_device* dev, const mvlm_buffer* qkv, mvlm_buffer* Kc, mvlm_buffer* Vc, mvlm_buffer* O,
                   int cached, int heads, int head_dim, float scale, const char* fn, Op* op) {
    REQUIRE(dev && qkv && Kc && Vc && O, "%s: null argument", fn);
    REQUIRE(qkv->dev == dev && Kc->dev == dev && Vc->dev == dev && O->dev == dev,
            "%s: buffers belong to another device", fn);
    REQUIRE(cached >= 0 && heads > 0 && head_dim > 0, "%s: cached=%d num_heads=%d head_dim=%d", fn, cached, heads,
            head_dim);
    REQUIRE(scale >= 0.0f && scale < INFINITY, "%s: scale %g must be finite and non-negative", fn, (double)scale);
    if (head_dim != 64 && head_dim != 128)
        return set_error(MVLM_ERR_UNSUPPORTED, "%s: head_dim=%d is not 64 or 128", fn, head_dim);
    if (heads > 192 || (int64_t)(cached + 1) * heads * head_dim * 2 > ((int64_t)1 << 31))
        return set_error(MVLM_ERR_UNSUPPORTED, "%s: more than 192 heads or a cache over 2 GiB", fn);
    REQUIRE(aligned16(qkv->ptr) && aligned16(Kc->ptr) && aligned16(Vc->ptr) && aligned16(O->ptr),
            "%s: qkv, K_cache, V_cache and O must be 16-byte aligned", fn);
    const size_t row = (size_t)heads * head_dim;
    NEED(qkv, 3 * row * 4, "qkv");
    NEED(Kc, ((size_t)cached + 1) * row * 2, "K_cache");
    NEED(Vc, ((size_t)cached + 1) * row * 2, "V_cache");
    NEED(O, row * 4, "O");
    REQUIRE(!(overlaps(Kc->ptr, Kc->bytes, Vc->ptr, Vc->bytes) || overlaps(O->ptr, row * 4, qkv->ptr, 3 * row * 4) ||
              overlaps(O->ptr, row * 4, Kc->ptr, Kc->bytes) || overlaps(O->ptr, row * 4, Vc->ptr, Vc->bytes)),
            "%s: K_cache, V_cache and O must not overlap each other or qkv", fn);
    op->kind = OP_ATTN_STEP;
    op->a = qkv->ptr; op->b = Kc->ptr; op->v = Vc->ptr; op->c = O->ptr;
    op->c_dtype = MVLM_F32;
    op->N = cached; op->batch = heads; op->K = head_dim;
    op->scale = scale == 0.0f ? 1.0f / sqrtf((float)head_dim) : scale;
    op->num_cus = dev->prop.multiProcessorCount;
    op->workspace_bytes = stream_attn_workspace_bytes(heads, head_dim, cached, 1, op->num_cus);
    return device_scratch(dev, op->workspace_bytes, &op->workspace);
}

static StreamAttnDesc attn_step_desc(const Op& op) {
    StreamAttnDesc d;
    d.qkv = op.a; d.k = const_cast<void*>(op.b); d.v = const_cast<void*>(op.v); d.o = (float*)op.c;
    d.heads = op.batch; d.head_dim = op.K; d.cached = op.N; d.mode = 1; d.step = 1; d.scale = op.scale;
    d.workspace = op.workspace;
    return d;
}

int make_argmax(mvlm_device* dev, const mvlm_buffer* x, int dtype, int rows, int n, int64_t ld,
                mvlm_buffer* out, const char* fn, Op* op) {
    REQUIRE(dev && x && out, "%s: null argument", fn);
    REQUIRE(x->dev == dev && out->dev == dev, "%s: buffers belong to another device", fn);
    REQUIRE(is_dense(dtype), "%s: dtype %d is not F32/F16/BF16", fn, dtype);
    REQUIRE(rows > 0 && n > 0 && ld >= n, "%s: rows=%d n=%d ld=%lld", fn, rows, n, (long long)ld);
    REQUIRE(rows <= (1 << 30), "%s: rows=%d too large", fn, rows);
    NEED(x, ((size_t)(rows - 1) * ld + n) * dtype_size(dtype), "x");
    NEED(out, (size_t)rows * 4, "out_index");
    REQUIRE(((uintptr_t)out->ptr & 3u) == 0 && ((uintptr_t)x->ptr % dtype_size(dtype)) == 0,
            "%s: misaligned buffer", fn);
    op->kind = OP_ARGMAX;
    op->a = x->ptr; op->c = out->ptr;
    op->a_dtype = dtype;
    op->M = rows; op->N = n; op->lda = ld;
    if (argmax_splits(rows, n) > 1) return device_sync_words(dev, &op->workspace);
    return MVLM_OK;
}

// Dense GEMV (M == 1) or dequantizing GEMV / skinny GEMM (M <= 16).
// want_dtype: required weight dtype, or -1 for any.
int make_gemv(mvlm_device* dev, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W, mvlm_buffer* y,
              int y_dtype, int M, int N, int K, int want_dtype, const char* fn, Op* op) {
    REQUIRE(dev && x && W && y, "%s: null argument", fn);
    REQUIRE(x->dev == dev && W->dev == dev && y->dev == dev, "%s: handles belong to another device", fn);
    if (want_dtype >= 0) REQUIRE(W->dtype == want_dtype, "%s: weight dtype %d, expected %d", fn, W->dtype, want_dtype);
    REQUIRE(N > 0 && K > 0, "%s: N=%d K=%d must be positive", fn, N, K);
    REQUIRE(W->N == N && W->K == K, "%s: weight is [%d x %d], call asks for N=%d K=%d", fn, W->N, W->K, N, K);
    REQUIRE(aligned16(x->ptr), "%s: x must be 16-byte aligned", fn);
    op->a = x->ptr; op->c = y->ptr; op->w = W;
    op->M = M; op->N = N; op->K = K;
    op->a_dtype = x_dtype; op->c_dtype = y_dtype;
    op->num_cus = dev->prop.multiProcessorCount;
    if (is_quant(W->dtype)) {
        REQUIRE(M >= 1 && M <= 16, "%s: M=%d outside [1, 16]", fn, M);
        REQUIRE(x_dtype == MVLM_F32 && y_dtype == MVLM_F32, "%s: quantized weights take fp32 x and y", fn);
        NEED(x, (size_t)M * K * 4, "x");
        NEED(y, (size_t)M * N * 4, "y");
        const bool streams = M == 1 ? stream_supported(W) : (M <= 4 && stream_supported(W, M));
        if (!streams && !skinny_supported(1, &W, op->num_cus))
            return set_error(MVLM_ERR_UNSUPPORTED, "%s: K=%d is outside the skinny kernel's range (a multiple of 32 "
                             "whose block scales fit in LDS, weight below 2 GiB)", fn, K);
        op->kind = OP_GEMV_QUANT;
        return MVLM_OK;
    }
    REQUIRE(M == 1, "%s: dense weights take M == 1 (M=%d); use mvlm_gemm_packed", fn, M);
    REQUIRE(is_dense(x_dtype) && is_dense(y_dtype), "%s: x/y dtypes must be F32/F16/BF16", fn);
    NEED(x, (size_t)K * dtype_size(x_dtype), "x");
    NEED(y, (size_t)N * dtype_size(y_dtype), "y");
    op->kind = OP_GEMV_DENSE;
    return MVLM_OK;
}

// Independent GEMVs (M = 1) or skinny GEMMs over quantized weights (M <= 16,
// fp32 x [M][K] and y [M][N] per entry) issued as one launch; quant_only
// refuses dense weights at M = 1 too.
int make_gemv_group(mvlm_device* dev, int M, int count, const mvlm_gemv_desc* descs, const char* fn, Op* op,
                    bool quant_only = false) {
    REQUIRE(dev && descs, "%s: null argument", fn);
    REQUIRE(count >= 1 && count <= MVLM_MAX_GROUP, "%s: count=%d outside [1, %d]", fn, count, MVLM_MAX_GROUP);
    REQUIRE(M >= 1 && M <= 16, "%s: M=%d outside [1, 16]", fn, M);
    for (int i = 0; i < count; ++i) {
        const mvlm_gemv_desc& d = descs[i];
        REQUIRE(d.W, "%s: entry %d has no weight", fn, i);
        REQUIRE(!quant_only || is_quant(d.W->dtype), "%s: entry %d weight dtype %d is not Q8_0/Q4_0", fn, i,
                d.W->dtype);
        Op one{};
        int st = make_gemv(dev, d.x, d.x_dtype, d.W, d.y, d.y_dtype, M, d.W->N, d.W->K, -1, fn, &one);
        if (st != MVLM_OK) return st;
        REQUIRE(d.W->dtype == descs[0].W->dtype, "%s: entry %d weight dtype %d differs from entry 0 (%d)", fn, i,
                d.W->dtype, descs[0].W->dtype);
        REQUIRE(d.x_dtype == descs[0].x_dtype, "%s: entry %d x dtype differs from entry 0", fn, i);
        if (M == 1 && !stream_supported(d.W))
            return set_error(MVLM_ERR_UNSUPPORTED, "%s: entry %d: rows of %lld bytes (K=%d) are outside the grouped "
                             "kernel's range (<= 16 KiB, K a multiple of the 16-byte vector, weight below 2 GiB)", fn, i,
                             (long long)weight_row_bytes(d.W), d.W->K);
        if (M > 1 && d.W->K % 32 != 0)
            return set_error(MVLM_ERR_UNSUPPORTED, "%s: entry %d: K=%d is not a multiple of 32", fn, i, d.W->K);
        op->gx[i] = d.x->ptr;
        op->gw[i] = d.W;
        op->gy[i] = d.y->ptr;
        op->gyd[i] = d.y_dtype;
    }
    op->kind = OP_GEMV_GROUP;
    op->gcount = count;
    op->M = M;
    op->a_dtype = descs[0].x_dtype;
    op->num_cus = dev->prop.multiProcessorCount;
    if (M > 1) {   // the skinny kernel serves the group unless every entry streams (launch_group_op)
        bool stream = M <= 4;
        for (int i = 0; i < count && stream; ++i) stream = stream_supported(op->gw[i], M);
        if (!stream && !skinny_supported(count, op->gw, op->num_cus))
            return set_error(MVLM_ERR_UNSUPPORTED, "%s: the group's block scales exceed the skinny kernel's LDS", fn);
    }
    return MVLM_OK;
}

// M > 1: the streaming kernel while every entry fits it (M <= 4), else the
// matrix-core skinny kernel.  with_attn: the launch also computes op.attn.
static hipError_t launch_group_op(hipStream_t s, const Op& op, bool with_attn) {
    if (op.M == 1)
        return launch_gemv_stream_group(s, op.gcount, op.gx, op.a_dtype, op.gw, op.gy, op.gyd, op.num_cus, op.gep, 1,
                                        with_attn ? &op.attn : nullptr);
    bool stream = op.M <= 4;
    for (int i = 0; i < op.gcount && stream; ++i) stream = stream_supported(op.gw[i], op.M);
    if (stream)
        return launch_gemv_stream_group(s, op.gcount, op.gx, op.a_dtype, op.gw, op.gy, op.gyd, op.num_cus, op.gep,
                                        op.M);
    const float* xs[MVLM_MAX_GROUP];
    float* ys[MVLM_MAX_GROUP];
    for (int i = 0; i < op.gcount; ++i) {
        xs[i] = (const float*)op.gx[i];
        ys[i] = (float*)op.gy[i];
    }
    return launch_gemm_skinny_group(s, op.M, op.gcount, xs, op.gw, ys, op.num_cus, op.gep);
}

// Per-entry epilogues of a grouped op (eps may be null: none).
int make_group_epilogues(mvlm_device* dev, const mvlm_epilogue* eps, const char* fn, Op* op) {
    if (!eps) return MVLM_OK;
    for (int i = 0; i < op->gcount; ++i) {
        const int st = make_epilogue(dev, &eps[i], op->M, op->gw[i]->N, op->gyd[i], fn, &op->gep[i]);
        if (st != MVLM_OK) return st;
    }
    return MVLM_OK;
}

hipError_t enqueue_op(hipStream_t s, const Op& op, bool with_attn = false) {
    switch (op.kind) {
        case OP_GEMV_GROUP:
            return launch_group_op(s, op, with_attn);
        case OP_GEMM_NAIVE:
            return launch_gemm_naive(s, (const uint16_t*)op.a, (const uint16_t*)op.b, (uint16_t*)op.c, op.M, op.N, op.K);
        case OP_GEMM_TILED:
            return launch_gemm_tiled(s, (const uint16_t*)op.a, (const uint16_t*)op.b, (uint16_t*)op.c, op.M, op.N, op.K);
        case OP_GEMV_EXACT:
            return launch_gemv_exact(s, (const uint16_t*)op.a, op.w, (uint16_t*)op.c);
        case OP_GEMM_MFMA:
            if (op.c_dtype == MVLM_F32 && !op.ep.any() &&
                smallk_supported(op.M, op.N, op.K, op.lda, op.ldb, op.ldc, op.sA, op.sB, op.a, op.b, op.c))
                return launch_gemm_smallk(s, op.a, op.a_dtype, op.b, (float*)op.c, op.batch, op.M, op.N, op.K, op.lda,
                                          op.ldb, op.sA, op.sB, op.sC, op.num_cus);
            return launch_gemm_mfma(s, op.a, op.a_dtype, op.b, op.c, op.c_dtype, op.batch, op.M, op.N, op.K,
                                    op.lda, op.ldb, op.ldc, op.sA, op.sB, op.sC, op.kread_b, op.num_cus, &op.ep,
                                    op.workspace, op.workspace_bytes);
        case OP_GEMV_DENSE:
            if (stream_supported(op.w))
                return launch_gemv_stream(s, op.a, op.a_dtype, op.w, op.c, op.c_dtype, op.num_cus, &op.ep);
            return launch_gemv_dense(s, op.a, op.a_dtype, op.w, op.c, op.c_dtype, op.N, op.K, &op.ep);
        case OP_GEMV_QUANT:
            if (op.M == 1 && stream_supported(op.w))
                return launch_gemv_stream(s, op.a, MVLM_F32, op.w, op.c, MVLM_F32, op.num_cus, &op.ep);
            if (op.M <= 4 && stream_supported(op.w, op.M))
                return launch_gemv_stream_batch(s, (const float*)op.a, op.w, (float*)op.c, op.M, op.num_cus, &op.ep);
            return launch_gemm_skinny(s, (const float*)op.a, op.w, (float*)op.c, op.M, op.N, op.K, op.num_cus,
                                      &op.ep);
        case OP_ARGMAX:
            return launch_argmax(s, op.a, op.a_dtype, op.M, op.N, op.lda, (int*)op.c, op.workspace);
        case OP_ATTENTION:
            return launch_attention(s, op.a, op.b, op.v, op.c, op.c_dtype, op.M, op.N, op.batch, op.K, op.causal,
                                    op.scale, op.num_cus, op.workspace, op.workspace_bytes);
        case OP_ATTN_STEP:
            return launch_attn_decode(s, attn_step_desc(op), op.num_cus);
    }
    return hipErrorInvalidValue;
}

int run_one(mvlm_device* dev, const Op& op, mvlm_event** ev, const char* fn) {
    LaunchScope ls(dev, ev);
    if (ls.status != MVLM_OK) return ls.status;
    hipError_t e = enqueue_op(dev->stream, op);
    if (e != hipSuccess) ls.status = check_hip(e, fn);
    return ls.finish(fn);
}

}  // namespace

// ---------------------------------------------------------------------------
// direct entry points
// ---------------------------------------------------------------------------

// the second step of a two-step op construction, run only if the first succeeded
template <class F>
int then(int st, F&& next) {
    return st != MVLM_OK ? st : next();
}

#define RUN(make_call)                                 \
    do {                                               \
        if (ev) *ev = nullptr;                         \
        Op op{};                                       \
        int st = (make_call);                          \
        if (st != MVLM_OK) return st;                  \
        return run_one(dev, op, ev, fn);               \
    } while (0)

extern "C" int mvlm_gemm_naive(mvlm_device* dev, const mvlm_buffer* A, const mvlm_buffer* B, mvlm_buffer* C,
                               int M, int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_ref_gemm(OP_GEMM_NAIVE, dev, A, B, C, M, N, K, fn, &op));
}

extern "C" int mvlm_gemm_tiled(mvlm_device* dev, const mvlm_buffer* A, const mvlm_buffer* B, mvlm_buffer* C,
                               int M, int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_ref_gemm(OP_GEMM_TILED, dev, A, B, C, M, N, K, fn, &op));
}

extern "C" int mvlm_gemv_exact(mvlm_device* dev, const mvlm_buffer* x, const mvlm_weight* W, mvlm_buffer* y,
                               int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemv_exact(dev, x, W, y, N, K, fn, &op));
}

extern "C" int mvlm_gemm_packed(mvlm_device* dev, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                                mvlm_buffer* C, int c_dtype, int M, int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemm_packed(dev, A, a_dtype, W, C, c_dtype, M, N, K, fn, &op));
}

extern "C" int mvlm_gemm_packed_ex(mvlm_device* dev, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                                   mvlm_buffer* C, int c_dtype, int M, int N, int K, const mvlm_epilogue* ep,
                                   mvlm_event** ev) {
    const char* fn = __func__;
    RUN(then(make_gemm_packed(dev, A, a_dtype, W, C, c_dtype, M, N, K, fn, &op),
             [&] { return make_epilogue(dev, ep, M, N, c_dtype, fn, &op.ep); }));
}

extern "C" int mvlm_gemm_packed_ex_noalloc(mvlm_device* dev, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                                           mvlm_buffer* C, int c_dtype, int M, int N, int K,
                                           const mvlm_epilogue* ep) {
    const char* fn = __func__;
    Op op{};
    int st = make_gemm_packed_op(dev, A, a_dtype, W, C, c_dtype, M, N, K, fn, &op);
    if (st == MVLM_OK) st = make_epilogue(dev, ep, M, N, c_dtype, fn, &op.ep);
    if (st != MVLM_OK) return st;
    if (op.workspace_bytes > (size_t)MVLM_NOALLOC_SCRATCH_BYTES)
        return set_error(MVLM_ERR_UNSUPPORTED, "%s: %dx%dx%d needs %zu bytes of workspace, above the %zu bytes this "
                         "entry point holds; use mvlm_gemm_packed_ex", fn, M, N, K, op.workspace_bytes,
                         (size_t)MVLM_NOALLOC_SCRATCH_BYTES);
    if (op.workspace_bytes > 0) {
        if (!dev->noalloc_scratch) return set_error(MVLM_ERR_HIP, "%s: the fixed workspace was not resolved", fn);
        op.workspace = dev->noalloc_scratch;
    }
    return run_one(dev, op, nullptr, fn);
}

extern "C" int mvlm_gemm_batched(mvlm_device* dev, const mvlm_buffer* A, const mvlm_buffer* B, mvlm_buffer* C,
                                 int batch, int M, int N, int K, int64_t lda, int64_t ldb, int64_t ldc,
                                 int64_t strideA, int64_t strideB, int64_t strideC, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemm_batched(dev, A, B, C, batch, M, N, K, lda, ldb, ldc, strideA, strideB, strideC, fn, &op));
}

extern "C" int mvlm_gemv(mvlm_device* dev, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W,
                         mvlm_buffer* y, int y_dtype, int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemv(dev, x, x_dtype, W, y, y_dtype, 1, N, K, -1, fn, &op));
}

extern "C" int mvlm_gemv_ex(mvlm_device* dev, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W,
                            mvlm_buffer* y, int y_dtype, int N, int K, const mvlm_epilogue* ep, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(then(make_gemv(dev, x, x_dtype, W, y, y_dtype, 1, N, K, -1, fn, &op),
             [&] { return make_epilogue(dev, ep, 1, N, y_dtype, fn, &op.ep); }));
}

extern "C" int mvlm_gemv_grouped(mvlm_device* dev, int count, const mvlm_gemv_desc* descs, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemv_group(dev, 1, count, descs, fn, &op));
}

extern "C" int mvlm_gemm_quant_grouped(mvlm_device* dev, int M, int count, const mvlm_gemv_desc* descs,
                                       mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemv_group(dev, M, count, descs, fn, &op, true));
}

extern "C" int mvlm_gemv_grouped_ex(mvlm_device* dev, int count, const mvlm_gemv_desc* descs,
                                    const mvlm_epilogue* eps, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(then(make_gemv_group(dev, 1, count, descs, fn, &op), [&] { return make_group_epilogues(dev, eps, fn, &op); }));
}

extern "C" int mvlm_gemm_quant_grouped_ex(mvlm_device* dev, int M, int count, const mvlm_gemv_desc* descs,
                                          const mvlm_epilogue* eps, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(then(make_gemv_group(dev, M, count, descs, fn, &op, true),
             [&] { return make_group_epilogues(dev, eps, fn, &op); }));
}

extern "C" int mvlm_gemv_q8_0(mvlm_device* dev, const mvlm_buffer* x, const mvlm_weight* W, mvlm_buffer* y,
                              int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemv(dev, x, MVLM_F32, W, y, MVLM_F32, 1, N, K, MVLM_Q8_0, fn, &op));
}

extern "C" int mvlm_gemv_q4_0(mvlm_device* dev, const mvlm_buffer* x, const mvlm_weight* W, mvlm_buffer* y,
                              int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemv(dev, x, MVLM_F32, W, y, MVLM_F32, 1, N, K, MVLM_Q4_0, fn, &op));
}

extern "C" int mvlm_gemm_q8_0(mvlm_device* dev, const mvlm_buffer* X, const mvlm_weight* W, mvlm_buffer* Y,
                              int M, int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemv(dev, X, MVLM_F32, W, Y, MVLM_F32, M, N, K, MVLM_Q8_0, fn, &op));
}

extern "C" int mvlm_gemm_q4_0(mvlm_device* dev, const mvlm_buffer* X, const mvlm_weight* W, mvlm_buffer* Y,
                              int M, int N, int K, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_gemv(dev, X, MVLM_F32, W, Y, MVLM_F32, M, N, K, MVLM_Q4_0, fn, &op));
}

extern "C" int mvlm_attention(mvlm_device* dev, const mvlm_buffer* Q, const mvlm_buffer* K, const mvlm_buffer* V,
                              mvlm_buffer* O, int o_dtype, int seq_q, int seq_kv, int num_heads, int head_dim,
                              int causal, float scale, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_attention(dev, Q, K, V, O, o_dtype, seq_q, seq_kv, num_heads, head_dim, causal, scale, fn, &op));
}

extern "C" int mvlm_attention_prefill(mvlm_device* dev, const mvlm_buffer* Q, const mvlm_buffer* K,
                                      const mvlm_buffer* V, mvlm_buffer* output, int seq_len, int num_heads,
                                      int head_dim, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_attention(dev, Q, K, V, output, MVLM_F16, seq_len, seq_len, num_heads, head_dim, 1, 0.0f, fn, &op));
}

extern "C" int mvlm_attention_decode(mvlm_device* dev, const mvlm_buffer* Q, const mvlm_buffer* K_cache,
                                     const mvlm_buffer* V_cache, mvlm_buffer* output, int cache_len, int num_heads,
                                     int head_dim, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_attention(dev, Q, K_cache, V_cache, output, MVLM_F16, 1, cache_len, num_heads, head_dim, 0, 0.0f, fn,
                       &op));
}

extern "C" int mvlm_attention_decode_step(mvlm_device* dev, const mvlm_buffer* qkv, mvlm_buffer* K_cache,
                                          mvlm_buffer* V_cache, mvlm_buffer* O, int cached, int num_heads,
                                          int head_dim, float scale, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_attn_step(dev, qkv, K_cache, V_cache, O, cached, num_heads, head_dim, scale, fn, &op));
}

extern "C" int mvlm_argmax(mvlm_device* dev, const mvlm_buffer* x, int dtype, int rows, int n, int64_t ld,
                           mvlm_buffer* out_index, mvlm_event** ev) {
    const char* fn = __func__;
    RUN(make_argmax(dev, x, dtype, rows, n, ld, out_index, fn, &op));
}

// ---------------------------------------------------------------------------
// plans
// ---------------------------------------------------------------------------

struct mvlm_plan {
    mvlm_device* dev = nullptr;
    std::vector<Op> ops;
    bool fuse = true;             // mvlm_plan_set_fusion
    std::vector<void*> sync_areas;   // of the fusable entries (SYNC_BYTES each)
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

static void drop_graph(mvlm_plan* p) {
    if (p->exec) (void)hipGraphExecDestroy(p->exec);
    if (p->graph) (void)hipGraphDestroy(p->graph);
    p->exec = nullptr;
    p->graph = nullptr;
}

extern "C" int mvlm_plan_create(mvlm_device* dev, mvlm_plan** out) {
    REQUIRE(dev && out, "mvlm_plan_create: null argument");
    *out = nullptr;
    mvlm_plan* p = new (std::nothrow) mvlm_plan();
    if (!p) return set_error(MVLM_ERR_OUT_OF_MEMORY, "plan allocation failed");
    p->dev = dev;
    *out = p;
    return MVLM_OK;
}

extern "C" int mvlm_plan_destroy(mvlm_plan* plan) {
    REQUIRE(plan, "mvlm_plan_destroy: plan is null");
    drop_graph(plan);
    if (!plan->sync_areas.empty()) {
        (void)hipSetDevice(plan->dev->ordinal);
        (void)hipStreamSynchronize(plan->dev->stream);
        for (void* p : plan->sync_areas) (void)hipFree(p);
    }
    delete plan;
    return MVLM_OK;
}

extern "C" int mvlm_plan_size(const mvlm_plan* plan) { return plan ? (int)plan->ops.size() : MVLM_ERR_INVALID_ARG; }

// Gives op (a grouped GEMV) attention d with a zeroed sync area of its own,
// if the launch can carry it (stream_attn_check).
static bool attach_sync(mvlm_plan* plan, Op& op, StreamAttnDesc d) {
    mvlm_device* dev = plan->dev;
    if (hipSetDevice(dev->ordinal) != hipSuccess || hipMalloc(&d.sync, SYNC_BYTES) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    bool ok = hipMemset(d.sync, 0, SYNC_BYTES) == hipSuccess &&
              stream_attn_check(op.gcount, op.gx, op.a_dtype, op.gw, op.gy, op.gyd, d, op.num_cus) == hipSuccess;
    if (ok) {
        try {
            plan->sync_areas.push_back(d.sync);
        } catch (...) {
            ok = false;
        }
    }
    if (!ok) {
        (void)hipGetLastError();
        (void)hipFree(d.sync);
        return false;
    }
    op.attn = d;
    return true;
}

// A grouped M = 1 GEMV pushed right after a decode attention (OP_ATTENTION
// with one query, fp32 output, head_dim 64 or 128; or OP_ATTN_STEP) that
// some entries read as x can carry that attention in its own launch, ahead of
// those entries.  The entries must not write the attention's inputs or
// output, nor read its output other than as x (nor, for a step, the caches),
// and the launch must fit the fused kernel (stream_attn_check).  Marks op and
// gives it the attention's description; the plan then skips the attention
// launch while fusion is on.  A step already carried by the GEMV before it
// moves here: measured, waiting readers cost less than a waiting attention.
static void mark_fusable(mvlm_plan* plan, Op& op) {
    if (op.kind != OP_GEMV_GROUP || op.M != 1 || op.a_dtype != MVLM_F32 || plan->ops.empty()) return;
    const Op& a = plan->ops.back();
    const bool step = a.kind == OP_ATTN_STEP;
    if (!step && (a.kind != OP_ATTENTION || a.M != 1 || a.c_dtype != MVLM_F32 || (a.K != 64 && a.K != 128))) return;
    const size_t row = (size_t)a.batch * a.K;
    const size_t in_bytes = step ? 3 * row * 4 : row * 2;                       // qkv or q
    const size_t kv_bytes = ((size_t)a.N + (step ? 1 : 0)) * row * 2;
    const size_t o_bytes = row * 4;
    bool reads_o = false;
    for (int i = 0; i < op.gcount; ++i) {
        const mvlm_weight* w = op.gw[i];
        const size_t y_bytes = (size_t)w->N * dtype_size(op.gyd[i]);
        if (overlaps(op.gy[i], y_bytes, a.a, in_bytes) || overlaps(op.gy[i], y_bytes, a.b, kv_bytes) ||
            overlaps(op.gy[i], y_bytes, a.v, kv_bytes) || overlaps(op.gy[i], y_bytes, a.c, o_bytes))
            return;
        const size_t x_bytes = (size_t)w->K * 4;
        if (op.gx[i] == a.c) reads_o = true;
        else if (overlaps(op.gx[i], x_bytes, a.c, o_bytes)) return;
        const Epilogue& e = op.gep[i];
        const size_t eb = (size_t)w->N * dtype_size(e.dtype);
        for (const void* in : {(const void*)e.bias, e.mul, e.res})
            if (overlaps(in, eb, a.c, o_bytes)) return;
        if (step)   // the step writes cache row `cached`: no entry may read the caches
            for (const void* in : {op.gx[i], (const void*)e.bias, e.mul, e.res}) {
                const size_t nb = in == op.gx[i] ? x_bytes : eb;
                if (overlaps(in, nb, a.b, kv_bytes) || overlaps(in, nb, a.v, kv_bytes)) return;
            }
    }
    if (!reads_o) return;
    StreamAttnDesc d;
    if (step) {
        d = attn_step_desc(a);
    } else {
        d.q = a.a; d.k = const_cast<void*>(a.b); d.v = const_cast<void*>(a.v); d.o = (float*)a.c;
        d.heads = a.batch; d.head_dim = a.K; d.cached = a.N; d.scale = a.scale;
        if (device_scratch(plan->dev, stream_attn_workspace_bytes(d.heads, d.head_dim, d.cached, 0, op.num_cus),
                           &d.workspace) != MVLM_OK)
            return;
    }
    d.mode = 0;
    if (!attach_sync(plan, op, d)) return;
    op.attn_carry = 1;
    if (step && plan->ops.size() >= 2 && plan->ops[plan->ops.size() - 2].attn_carry == 2)
        plan->ops[plan->ops.size() - 2].attn_carry = 0;   // no longer carried by the producer's launch
}

// A decode attention step (OP_ATTN_STEP) pushed right after a grouped M = 1
// GEMV one of whose entries writes its qkv (fp32, N = 3 heads D) can run in
// that GEMV's launch, after that entry's rows.  The other entries must not
// write qkv, the caches or O, and no entry may read the caches or O (the
// step writes cache row `cached` and O).  Marks the GEMV entry.
static void mark_fusable_after(mvlm_plan* plan, const Op& a) {
    if (a.kind != OP_ATTN_STEP || plan->ops.empty()) return;
    Op& op = plan->ops.back();
    if (op.kind != OP_GEMV_GROUP || op.M != 1 || op.attn_carry != 0) return;
    const size_t row = (size_t)a.batch * a.K;
    const size_t kv_bytes = ((size_t)a.N + 1) * row * 2;
    int producers = 0;
    for (int i = 0; i < op.gcount; ++i) {
        const mvlm_weight* w = op.gw[i];
        const size_t y_bytes = (size_t)w->N * dtype_size(op.gyd[i]);
        const size_t x_bytes = (size_t)w->K * dtype_size(op.a_dtype);
        if (op.gy[i] == a.a && op.gyd[i] == MVLM_F32 && (size_t)w->N == 3 * row) {
            ++producers;
        } else if (overlaps(op.gy[i], y_bytes, a.a, 3 * row * 4)) {
            return;
        }
        if (overlaps(op.gy[i], y_bytes, a.b, kv_bytes) || overlaps(op.gy[i], y_bytes, a.v, kv_bytes) ||
            overlaps(op.gy[i], y_bytes, a.c, row * 4))
            return;
        const Epilogue& e = op.gep[i];
        const size_t eb = (size_t)w->N * dtype_size(e.dtype);
        for (const void* in : {op.gx[i], e.bias, e.mul, e.res}) {
            const size_t nb = in == op.gx[i] ? x_bytes : eb;
            if (overlaps(in, nb, a.b, kv_bytes) || overlaps(in, nb, a.v, kv_bytes) || overlaps(in, nb, a.c, row * 4))
                return;
        }
    }
    if (producers != 1) return;
    StreamAttnDesc d = attn_step_desc(a);
    if (attach_sync(plan, op, d)) op.attn_carry = 2;
}

static int plan_push(mvlm_plan* plan, Op op) {
    drop_graph(plan);   // a recorded graph no longer matches
    mark_fusable(plan, op);
    mark_fusable_after(plan, op);
    try {
        plan->ops.push_back(op);
    } catch (...) {
        return set_error(MVLM_ERR_OUT_OF_MEMORY, "plan growth failed");
    }
    return MVLM_OK;
}

extern "C" int mvlm_plan_add_gemv(mvlm_plan* plan, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W,
                                  mvlm_buffer* y, int y_dtype, int M) {
    const char* fn = __func__;
    REQUIRE(plan && W, "%s: null argument", fn);
    Op op{};
    int st = make_gemv(plan->dev, x, x_dtype, W, y, y_dtype, M, W->N, W->K, -1, fn, &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_gemv_ex(mvlm_plan* plan, const mvlm_buffer* x, int x_dtype, const mvlm_weight* W,
                                     mvlm_buffer* y, int y_dtype, const mvlm_epilogue* ep) {
    const char* fn = __func__;
    REQUIRE(plan && W, "%s: null argument", fn);
    Op op{};
    int st = make_gemv(plan->dev, x, x_dtype, W, y, y_dtype, 1, W->N, W->K, -1, fn, &op);
    if (st == MVLM_OK) st = make_epilogue(plan->dev, ep, 1, W->N, y_dtype, fn, &op.ep);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_gemm_packed_ex(mvlm_plan* plan, const mvlm_buffer* A, int a_dtype,
                                            const mvlm_weight* W, mvlm_buffer* C, int c_dtype, int M,
                                            const mvlm_epilogue* ep) {
    const char* fn = __func__;
    REQUIRE(plan && W, "%s: null argument", fn);
    Op op{};
    int st = make_gemm_packed(plan->dev, A, a_dtype, W, C, c_dtype, M, W->N, W->K, fn, &op);
    if (st == MVLM_OK) st = make_epilogue(plan->dev, ep, M, W->N, c_dtype, fn, &op.ep);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_gemv_grouped(mvlm_plan* plan, int count, const mvlm_gemv_desc* descs) {
    const char* fn = __func__;
    REQUIRE(plan, "%s: null argument", fn);
    Op op{};
    int st = make_gemv_group(plan->dev, 1, count, descs, fn, &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_gemm_quant_grouped(mvlm_plan* plan, int M, int count, const mvlm_gemv_desc* descs) {
    const char* fn = __func__;
    REQUIRE(plan, "%s: null argument", fn);
    Op op{};
    int st = make_gemv_group(plan->dev, M, count, descs, fn, &op, true);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_gemv_grouped_ex(mvlm_plan* plan, int count, const mvlm_gemv_desc* descs,
                                             const mvlm_epilogue* eps) {
    const char* fn = __func__;
    REQUIRE(plan, "%s: null argument", fn);
    Op op{};
    int st = make_gemv_group(plan->dev, 1, count, descs, fn, &op);
    if (st == MVLM_OK) st = make_group_epilogues(plan->dev, eps, fn, &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_gemm_quant_grouped_ex(mvlm_plan* plan, int M, int count, const mvlm_gemv_desc* descs,
                                                   const mvlm_epilogue* eps) {
    const char* fn = __func__;
    REQUIRE(plan, "%s: null argument", fn);
    Op op{};
    int st = make_gemv_group(plan->dev, M, count, descs, fn, &op, true);
    if (st == MVLM_OK) st = make_group_epilogues(plan->dev, eps, fn, &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_gemm_packed(mvlm_plan* plan, const mvlm_buffer* A, int a_dtype, const mvlm_weight* W,
                                         mvlm_buffer* C, int c_dtype, int M) {
    const char* fn = __func__;
    REQUIRE(plan && W, "%s: null argument", fn);
    Op op{};
    int st = make_gemm_packed(plan->dev, A, a_dtype, W, C, c_dtype, M, W->N, W->K, fn, &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_gemm_batched(mvlm_plan* plan, const mvlm_buffer* A, const mvlm_buffer* B,
                                          mvlm_buffer* C, int batch, int M, int N, int K, int64_t lda,
                                          int64_t ldb, int64_t ldc, int64_t strideA, int64_t strideB,
                                          int64_t strideC) {
    const char* fn = __func__;
    REQUIRE(plan, "%s: null argument", fn);
    Op op{};
    int st = make_gemm_batched(plan->dev, A, B, C, batch, M, N, K, lda, ldb, ldc, strideA, strideB, strideC, fn, &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_attention(mvlm_plan* plan, const mvlm_buffer* Q, const mvlm_buffer* K,
                                       const mvlm_buffer* V, mvlm_buffer* O, int o_dtype, int seq_q, int seq_kv,
                                       int num_heads, int head_dim, int causal, float scale) {
    const char* fn = __func__;
    REQUIRE(plan, "%s: null argument", fn);
    Op op{};
    int st = make_attention(plan->dev, Q, K, V, O, o_dtype, seq_q, seq_kv, num_heads, head_dim, causal, scale, fn,
                            &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_attention_decode_step(mvlm_plan* plan, const mvlm_buffer* qkv, mvlm_buffer* K_cache,
                                                   mvlm_buffer* V_cache, mvlm_buffer* O, int cached, int num_heads,
                                                   int head_dim, float scale) {
    const char* fn = __func__;
    REQUIRE(plan, "%s: null argument", fn);
    Op op{};
    int st = make_attn_step(plan->dev, qkv, K_cache, V_cache, O, cached, num_heads, head_dim, scale, fn, &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

extern "C" int mvlm_plan_add_argmax(mvlm_plan* plan, const mvlm_buffer* x, int dtype, int rows, int n, int64_t ld,
                                    mvlm_buffer* out_index) {
    const char* fn = __func__;
    REQUIRE(plan, "%s: null argument", fn);
    Op op{};
    int st = make_argmax(plan->dev, x, dtype, rows, n, ld, out_index, fn, &op);
    return st != MVLM_OK ? st : plan_push(plan, op);
}

// Whether entry i is launched by a neighbour (a decode attention carried by
// the grouped GEMV after it, or a decode step by the one before it) and
// whether entry i carries a neighbour.
static bool carried(const mvlm_plan* plan, size_t i) {
    return plan->fuse && ((i + 1 < plan->ops.size() && plan->ops[i + 1].attn_carry == 1) ||
                          (i > 0 && plan->ops[i - 1].attn_carry == 2));
}
static bool carries(const mvlm_plan* plan, size_t i) { return plan->fuse && plan->ops[i].attn_carry != 0; }

// The plan's launches in order: one per entry, except attention entries
// carried by the next entry's launch.
static int enqueue_all(mvlm_plan* plan) {
    for (size_t i = 0; i < plan->ops.size(); ++i) {
        if (carried(plan, i)) continue;
        const hipError_t e = enqueue_op(plan->dev->stream, plan->ops[i], carries(plan, i));
        if (e != hipSuccess) return check_hip(e, "plan launch");
    }
    return MVLM_OK;
}

extern "C" int mvlm_plan_set_fusion(mvlm_plan* plan, int enable) {
    REQUIRE(plan, "mvlm_plan_set_fusion: plan is null");
    if (plan->fuse != (enable != 0)) drop_graph(plan);
    plan->fuse = enable != 0;
    return MVLM_OK;
}

extern "C" int mvlm_plan_fused(const mvlm_plan* plan) {
    if (!plan) return MVLM_ERR_INVALID_ARG;
    int n = 0;
    for (size_t i = 0; i < plan->ops.size(); ++i) n += carries(plan, i) ? 1 : 0;
    return n;
}

extern "C" int mvlm_plan_check(mvlm_plan* plan) {
    REQUIRE(plan, "mvlm_plan_check: plan is null");
    mvlm_device* dev = plan->dev;
    HIP_TRY(hipSetDevice(dev->ordinal));
    HIP_TRY(hipStreamSynchronize(dev->stream));
    int failed = 0;
    for (const Op& op : plan->ops) {
        if (!op.attn_carry) continue;
        uint32_t err = 0;
        HIP_TRY(hipMemcpy(&err, (const char*)op.attn.sync + SYNC_ERR_OFFSET, 4, hipMemcpyDeviceToHost));
        if (!err) continue;
        ++failed;
        HIP_TRY(hipMemset(op.attn.sync, 0, SYNC_BYTES));   // counters the failed launch left part-way
    }
    if (!failed) return MVLM_OK;
    return set_error(MVLM_ERR_HIP, "mvlm_plan_check: %d fused launch site(s) gave up waiting for their attention "
                     "after 20 ms; the workgroups that waited stored NaN", failed);
}

extern "C" int mvlm_plan_use_graph(mvlm_plan* plan, int enable) {
    REQUIRE(plan, "mvlm_plan_use_graph: plan is null");
    drop_graph(plan);
    if (!enable) return MVLM_OK;
    REQUIRE(!plan->ops.empty(), "mvlm_plan_use_graph: the plan is empty");
    hipStream_t s = plan->dev->stream;
    HIP_TRY(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    int st = enqueue_all(plan);
    hipGraph_t g = nullptr;
    int st2 = check_hip(hipStreamEndCapture(s, &g), "hipStreamEndCapture");
    if (st == MVLM_OK) st = st2;
    if (st != MVLM_OK) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    plan->graph = g;
    st = check_hip(hipGraphInstantiate(&plan->exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    if (st != MVLM_OK) drop_graph(plan);
    return st;
}

extern "C" int mvlm_plan_run(mvlm_plan* plan, int repeats, mvlm_event** ev) {
    if (ev) *ev = nullptr;
    REQUIRE(plan, "mvlm_plan_run: plan is null");
    REQUIRE(repeats >= 1, "mvlm_plan_run: repeats=%d must be positive", repeats);
    LaunchScope ls(plan->dev, ev);
    if (ls.status != MVLM_OK) return ls.status;
    for (int r = 0; r < repeats && ls.status == MVLM_OK; ++r) {
        if (plan->exec)
            ls.status = check_hip(hipGraphLaunch(plan->exec, plan->dev->stream), "hipGraphLaunch");
        else
            ls.status = enqueue_all(plan);
    }
    return ls.finish("plan run");
}

extern "C" int mvlm_plan_profile(mvlm_plan* plan, float* op_ms, int capacity) {
    REQUIRE(plan && op_ms, "mvlm_plan_profile: null argument");
    const int n = (int)plan->ops.size();
    REQUIRE(capacity >= n, "mvlm_plan_profile: capacity %d below the plan size %d", capacity, n);
    // two events per launch, attached to the kernel's own dispatch packet
    std::vector<hipEvent_t> ev(2 * (size_t)n, nullptr);
    int st = MVLM_OK;
    for (size_t i = 0; i < ev.size() && st == MVLM_OK; ++i) st = check_hip(hipEventCreate(&ev[i]), "hipEventCreate");
    hipStream_t s = plan->dev->stream;
    KernelTiming& t = kernel_timing();
    int launched = 0;
    int last = -1;
    for (int i = 0; i < n && st == MVLM_OK; ++i) {
        if (carried(plan, (size_t)i)) continue;   // timed with the launch that carries it
        t.start = ev[2 * i];
        t.stop = ev[2 * i + 1];
        const hipError_t e = enqueue_op(s, plan->ops[i], carries(plan, (size_t)i));
        t = KernelTiming{};
        if (e != hipSuccess) st = check_hip(e, "plan launch");
        else last = i;
    }
    t = KernelTiming{};
    launched = last + 1;
    if (st == MVLM_OK && launched > 0)
        st = check_hip(hipEventSynchronize(ev[2 * (size_t)(launched - 1) + 1]), "hipEventSynchronize");
    for (int i = 0; i < n && st == MVLM_OK; ++i) {
        if (carried(plan, (size_t)i)) op_ms[i] = 0.0f;
        else st = check_hip(hipEventElapsedTime(&op_ms[i], ev[2 * i], ev[2 * i + 1]), "hipEventElapsedTime");
    }
    for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);
    return st;
}
