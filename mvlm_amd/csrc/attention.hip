// Fused multi-head attention on CDNA4 matrix cores:
//   O[q][h][:] = sum_k softmax_k(scale * Q[q][h][:] . K[k][h][:] + mask) V[k][h][:]
// Q, K, V fp16 [seq][heads][head_dim] (the layout of src/kernels/attention.cl:44-56),
// fp32 scores and softmax, O fp16 or fp32.
//
// Replaces attention_prefill (src/kernels/attention.cl:46-179) and
// attention_decode (:197-295), which give one (query, head) pair a workgroup
// and recompute every Q.K dot product three times (max pass, sum pass,
// weighted-V pass), and the QK^T / softmax / PV round trips through HBM of an
// unfused version (the 16 x 729 x 729 fp32 score tensor of a SigLIP layer is
// 34 MB).  Scores never leave registers:
//  * a block owns 32 queries of one head; its NW waves split the keys
//    (wave w takes key tiles w, w + NW, ... of 32 keys) and each keeps an
//    online softmax (running max and sum, rescaled output accumulator); the
//    block merges the NW partial results through LDS at the end;
//  * S^T = K Q^T per tile: v_mfma_f32_32x32x16_f16 with A = the K tile (from
//    the wave's LDS) and B = Q (registers for the whole kernel); lane l's
//    accumulator column is query l%32 and register r is key
//    8(r/4) + 4(l/32) + r%4, so a query's softmax statistics are per lane
//    (plus one exchange with lane l^32);
//  * O^T = V^T P^T: A = V^T, B = the lane's own probabilities packed to
//    fp16: register r's key order above is taken as the k order of the
//    product, so A holds keys {4h..4h+3, 8+4h..8+4h+3} (+16 per k-step) to
//    match, and no data moves between lanes.  V is stored row-major in LDS
//    (like K) and its transposed fragments come from ds_read_b64_tr_b16
//    (within 16 lanes, lane j receives element j%4 of the 4-element rows read
//    by lanes 4k + j/4, k = 0..3): lane 4k + q reads 4 dims at 4q of key k, so
//    lane j gets dim j of 4 consecutive keys;
//  * the output accumulator O^T also has query l%32 per lane, so the online
//    rescaling is one multiply per register;
//  * every wave stages its own tiles (no block barrier in the key loop) and
//    loads tile j+1 into registers while it computes tile j.
// head_dim is padded to 16 KS (S^T k-steps) and 32 DT (O^T row tiles); the K
// tile's padding columns are zeroed once, V's columns past head_dim (never
// written) only feed output rows that are never stored.  Keys past the end
// read as zeros (buffer bounds check) and get score -inf.  Causal masking hides key k from query q
// when k > q + (seq_kv - seq_q) (queries aligned to the end of the keys;
// seq_q == seq_kv gives attention.cl's k > q) and skips the key tiles past
// the block's last query.
#include "common.h"
#include "device_math.h"

#include <algorithm>
#include <cstdlib>

namespace mvlm {

struct AttnArgs {
    const uint16_t* Q;
    const uint16_t* K;
    const uint16_t* V;
    void* O;
    int o_dtype;
    int seq_q, seq_kv, heads, D;
    int causal;
    float scale_log2;      // scale * log2(e): scores are kept in the exp2 domain
    // split over keys (blockIdx.z = split): each split covers tiles_per_split
    // key tiles and, when splits > 1, parks (m, l) and the unnormalized output
    // in ws for attention_combine_kernel
    int splits, tiles_per_split;
    float* ws;
};

// Partial results of split s for (query q, head h), record r = (s seq_q + q) heads + h:
// ws[r D ..] = D floats of unnormalized output; after all splits seq_q heads
// records, ws[.. + 2 r], [.. + 2 r + 1] = running max (exp2 domain) and sum.
__device__ __forceinline__ int64_t attn_record(const AttnArgs& a, int split, int q, int head) {
    return ((int64_t)split * a.seq_q + q) * a.heads + head;
}
__device__ __forceinline__ float* attn_ws_out(const AttnArgs& a, int64_t r) { return a.ws + r * a.D; }
__device__ __forceinline__ float* attn_ws_ml(const AttnArgs& a, int64_t r) {
    return a.ws + (int64_t)a.splits * a.seq_q * a.heads * a.D + 2 * r;
}

template <int KS, int DT>
struct AttnLayout {
    static constexpr int KROW = 16 * KS + 8;                  // K tile row pitch (halfs): odd multiple of 16 B
    // V tile row pitch (halfs): >= 32 DT (the transposed reads reach dim 32 DT - 1)
    // and 32 mod 64, so the 4 key rows a 32-lane half of a transposed read
    // touches start 16 banks apart (64 contiguous bytes each: all 64 banks)
    static constexpr int VP = DT == 1 ? 32 : DT <= 3 ? 96 : 160;
    static constexpr int STAGE = 32 * KROW * 2 + 32 * VP * 2;
    static constexpr int OPITCH = 32 * DT + 4;                // merge area row pitch (floats)
    static constexpr int MERGE = 32 * OPITCH * 4 + 2 * 32 * 4;
    static constexpr int REGION = ((STAGE > MERGE ? STAGE : MERGE) + 15) / 16 * 16;   // bytes per wave
    static constexpr int VI = (32 * DT + 63) / 64;            // quad-chunk rounds per tile (D <= 32 DT)
};

constexpr int ATTN_LDS_MAX = 160 * 1024;

__device__ __forceinline__ f32x16 mfma_f16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
}

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// two fp32 values to packed fp16, round to nearest even (one v_cvt_pk_f16_f32)
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
}

template <int KS, int DT, int NW>
__global__ __launch_bounds__(64 * NW) void attention_kernel(const AttnArgs a) {
    using L = AttnLayout<KS, DT>;
    constexpr int VI = L::VI;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int head = blockIdx.y;
    const int qb0 = blockIdx.x * 32;                      // block's first query
    const int q = qb0 + l32;                              // this lane's query
    const int D = a.D;
    const int64_t row = (int64_t)a.heads * D;             // elements between consecutive positions

    uint8_t* region = lds + wave * L::REGION;
    uint16_t* ks = (uint16_t*)region;                     // [32 keys][KROW]
    uint16_t* vt = (uint16_t*)(region + 32 * L::KROW * 2);   // [32 keys][VP]

    // zero the K tile's padding columns D .. 16 KS once (contracted with Q's
    // zeros): D is a multiple of 8, so whole 16-byte chunks, one row per lane
    if (lane < 32)
        for (int d = D; d < 16 * KS; d += 8) *reinterpret_cast<u32x4*>(ks + lane * L::KROW + d) = u32x4{0u, 0u, 0u, 0u};

    // Raw buffer loads: an offset at or past num_records reads zeros, which
    // covers keys past seq_kv, queries past seq_q and the idle lanes of a
    // partial chunk round (offset 2^31) without branches around the loads.
    const int row2 = (int)(row * 2);                      // bytes between consecutive positions
    const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc((void*)a.Q, 0, a.seq_q * row2, 0x00020000);
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc((void*)a.K, 0, a.seq_kv * row2, 0x00020000);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc((void*)a.V, 0, a.seq_kv * row2, 0x00020000);
    constexpr uint32_t OOB = 0x80000000u;

    // Q fragments of this lane: Q[q][head][16 s + 8 h .. +7], zero past D / seq_q
    u32x4 qf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int d = 16 * s + 8 * h;
        const uint32_t off = q < a.seq_q && d < D ? (uint32_t)(q * row2 + (head * D + d) * 2) : OOB;
        qf[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, (int)off, 0, 0));
    }

    const int shift = a.seq_kv - a.seq_q;
    const int last_key = a.causal ? min(a.seq_kv - 1, q + shift) : a.seq_kv - 1;   // lane's last visible key
    // keys below this are visible to every query of the block
    const int open_end = a.causal ? min(a.seq_kv, qb0 + shift + 1) : a.seq_kv;
    int kv_end = a.seq_kv;
    if (a.causal) kv_end = min(a.seq_kv, min(qb0 + 32, a.seq_q) + shift);

    // lane chunk c = lane + 64 i (c < D): keys 4 (c / cpr) .. +3, dims 8 (c % cpr) .. +7
    // with cpr = D / 8 chunks per row; consecutive lanes take consecutive
    // 16-byte chunks of one row, so each quad of lanes reads one 64-byte run
    const int cpr = D / 8;
    uint32_t coff[VI];
    int ckey[VI], cdim[VI];
#pragma unroll
    for (int i = 0; i < VI; ++i) {
        const int c = lane + 64 * i;
        ckey[i] = 4 * (c / cpr);
        cdim[i] = 8 * (c % cpr);
        coff[i] = c < D ? (uint32_t)(ckey[i] * row2 + (head * D + cdim[i]) * 2) : OOB;
    }
    u32x4 tk[VI][4], tv[VI][4];
    auto load_tile = [&](int kv0) {
        const uint32_t base = (uint32_t)(kv0 * row2);
#pragma unroll
        for (int i = 0; i < VI; ++i)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int off = (int)(coff[i] + base + u * row2);
                tk[i][u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
                tv[i][u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0));
            }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const int c = lane + 64 * i;
            if (64 * i + 64 <= D || c < D) {
                const int key0 = ckey[i], d = cdim[i];
#pragma unroll
                for (int u = 0; u < 4; ++u) *reinterpret_cast<u32x4*>(ks + (key0 + u) * L::KROW + d) = tk[i][u];
#pragma unroll
                for (int u = 0; u < 4; ++u) *reinterpret_cast<u32x4*>(vt + (key0 + u) * L::VP + d) = tv[i][u];
            }
        }
    };

    float mrun = -INFINITY, lrun = 0.0f;
    f32x16 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[t][r] = 0.0f;

    // This block's keys: tiles [split * tiles_per_split, +tiles_per_split) below kv_end.
    // Tiles past the end are still loaded (as zeros or spare rows) so the loop
    // body has no branch around its loads: the one in flight is never stored.
    const int split = blockIdx.z;
    const int kv_stop = min(kv_end, 32 * (split + 1) * a.tiles_per_split);
    int kv0 = 32 * (split * a.tiles_per_split + wave);
    load_tile(kv0);
    while (kv0 < kv_stop) {
        store_tile();
        const int kv_next = kv0 + 32 * NW;
        load_tile(kv_next);                               // in flight while this tile computes
        // this wave's own LDS: its stores above precede these reads in the wave's LDS order
        asm volatile("" ::: "memory");

        f32x16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
        for (int st = 0; st < KS; ++st) {
            const u32x4 kf = *reinterpret_cast<const u32x4*>(ks + l32 * L::KROW + 16 * st + 8 * h);
            s = mfma_f16(kf, qf[st], s);
        }
        // raw dot products; the scale (> 0) is applied inside the exponent
        if (kv0 + 32 > open_end) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kv0 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (key > last_key) s[r] = -INFINITY;
            }
        }
        float tmax = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, s[r]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64)) * a.scale_log2;
        // Lazy rescaling: the reference point mrun moves only when a score
        // exceeds it by more than 8 (probabilities stay <= 2^8, exact range
        // for fp16), so most tiles skip the accumulator rescale.
        if (__builtin_amdgcn_ballot_w64(tmax > mrun + 8.0f)) {
            const float mnew = fmaxf(mrun, tmax);
            // 0 when mrun = -inf; a lane that still sees no key keeps its zeros
            const float factor = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(mrun - mnew);
            lrun *= factor;
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[t][r] *= factor;
            mrun = mnew;
        }
        // mrun stays -inf while every key so far is hidden from this query
        const float msafe = mrun == -INFINITY ? 0.0f : mrun;
        float psum = 0.0f;
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], a.scale_log2, -msafe));
            psum += p[r];
        }
        psum += __shfl_xor(psum, 32, 64);
        lrun += psum;

        // O^T += V^T P^T over the tile's two 16-key steps
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            u32x4 pb;
#pragma unroll
            for (int j = 0; j < 4; ++j) pb[j] = pack_f16x2(p[8 * kk + 2 * j], p[8 * kk + 2 * j + 1]);
            // lane l: dim 32t + l%32 of keys 16kk + 4h + 0..3 (lo) and +8 (hi):
            // within its 16-lane group it reads key (l&15)>>2, dims 4(l&3)..+3
            // of the group's 16 (l>>4 selects the half of the 32-dim tile)
            const uint16_t* vgrp = vt + (16 * kk + 4 * h + ((lane & 15) >> 2)) * L::VP + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                lds_i16x4* p0 = (lds_i16x4*)(uintptr_t)lds_offset(vgrp + 32 * t);
                lds_i16x4* p1 = (lds_i16x4*)(uintptr_t)lds_offset(vgrp + 32 * t + 8 * L::VP);
                const u32x2 lo = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(p0));
                const u32x2 hi = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(p1));
                oacc[t] = mfma_f16(u32x4{lo[0], lo[1], hi[0], hi[1]}, pb, oacc[t]);
            }
        }
        asm volatile("" ::: "memory");                  // the next tile's stores follow these reads
        kv0 = kv_next;
    }

    auto store4 = [&](int qq, int d, float v0, float v1, float v2, float v3) {
        const int64_t off = (int64_t)qq * row + head * D + d;
        if (a.o_dtype == MVLM_F32)
            *reinterpret_cast<f32x4*>((float*)a.O + off) = f32x4{v0, v1, v2, v3};
        else
            *reinterpret_cast<u32x2*>((uint16_t*)a.O + off) = u32x2{pack_f16x2(v0, v1), pack_f16x2(v2, v3)};
    };

    if constexpr (NW == 1) {
        if (q >= a.seq_q) return;
        if (a.splits > 1) {
            const int64_t r = attn_record(a, split, q, head);
            float* wo = attn_ws_out(a, r);
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * t + 8 * g + 4 * h;
                    if (d < D)
                        *reinterpret_cast<f32x4*>(wo + d) =
                            f32x4{oacc[t][4 * g], oacc[t][4 * g + 1], oacc[t][4 * g + 2], oacc[t][4 * g + 3]};
                }
            if (h == 0) *reinterpret_cast<f32x2*>(attn_ws_ml(a, r)) = f32x2{mrun, lrun};
            return;
        }
        const float inv = 1.0f / lrun;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * t + 8 * g + 4 * h;      // registers 4g .. 4g+3: dims d .. d+3
                if (d < D)
                    store4(q, d, oacc[t][4 * g] * inv, oacc[t][4 * g + 1] * inv, oacc[t][4 * g + 2] * inv,
                           oacc[t][4 * g + 3] * inv);
            }
    } else {
        // merge the NW partial softmaxes: each wave parks (m, l, unnormalized O)
        // in its own region, then the block combines them per (query, 4 dims)
        float* om = (float*)region;                       // [32 queries][OPITCH]
        float* ml = om + 32 * L::OPITCH;                  // m[32], l[32]
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = 32 * t + 8 * g + 4 * h;
                *reinterpret_cast<f32x4*>(om + l32 * L::OPITCH + d) =
                    f32x4{oacc[t][4 * g], oacc[t][4 * g + 1], oacc[t][4 * g + 2], oacc[t][4 * g + 3]};
            }
        if (h == 0) {
            ml[l32] = mrun;
            ml[32 + l32] = lrun;
        }
        __syncthreads();
        for (int it = threadIdx.x; it < 32 * (D / 4); it += 64 * NW) {
            const int ql = it & 31, d = 4 * (it >> 5);
            if (qb0 + ql >= a.seq_q) continue;
            float mw[NW], mx = -INFINITY;
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                mw[w] = ((const float*)(lds + w * L::REGION))[32 * L::OPITCH + ql];
                mx = fmaxf(mx, mw[w]);
            }
            // a split's keys may all be hidden from a query (causal): m = -inf in
            // every wave; the record then keeps m = -inf with l = 0, O = 0
            const float mref = mx == -INFINITY ? 0.0f : mx;
            float lsum = 0.0f;
            f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float* rw = (const float*)(lds + w * L::REGION);
                const float f = __builtin_amdgcn_exp2f(mw[w] - mref);
                lsum += f * rw[32 * L::OPITCH + 32 + ql];
                o += f * *reinterpret_cast<const f32x4*>(rw + ql * L::OPITCH + d);
            }
            if (a.splits > 1) {
                const int64_t r = attn_record(a, split, qb0 + ql, head);
                *reinterpret_cast<f32x4*>(attn_ws_out(a, r) + d) = o;
                if (d == 0) *reinterpret_cast<f32x2*>(attn_ws_ml(a, r)) = f32x2{mx, lsum};
                continue;
            }
            const float inv = 1.0f / lsum;
            store4(qb0 + ql, d, o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
        }
    }
}

// Merges the splits' partial softmaxes: thread = (query, head, 4 dims).  The
// records are read 16 at a time (all loads in flight together; the split
// count is at most 32) and folded in with an online rescale, so no pass over
// the maxima comes first.
__global__ __launch_bounds__(256) void attention_combine_kernel(const AttnArgs a) {
    constexpr int BATCH = 16;
    const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int d4 = a.D / 4;
    if (item >= (int64_t)a.seq_q * a.heads * d4) return;
    const int64_t qh = item / d4;                          // q * heads + head
    const int d = 4 * (int)(item - qh * d4);
    const int64_t stride = (int64_t)a.seq_q * a.heads;     // records between splits
    float mx = -INFINITY, lsum = 0.0f;
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < a.splits; s0 += BATCH) {
        f32x2 ml[BATCH];
        f32x4 ov[BATCH];
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            const int64_t r = min(s0 + u, a.splits - 1) * stride + qh;
            ml[u] = *reinterpret_cast<const f32x2*>(attn_ws_ml(a, r));
            ov[u] = *reinterpret_cast<const f32x4*>(attn_ws_out(a, r) + d);
        }
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
            if (s0 + u >= a.splits || ml[u][0] == -INFINITY) continue;   // past the end, or saw no key
            const float mn = fmaxf(mx, ml[u][0]);
            const float f_old = __builtin_amdgcn_exp2f(mx - mn);          // 0 while mx = -inf
            const float f_new = __builtin_amdgcn_exp2f(ml[u][0] - mn);
            lsum = lsum * f_old + f_new * ml[u][1];
            o = o * f_old + f_new * ov[u];
            mx = mn;
        }
    }
    const float inv = 1.0f / lsum;
    const int64_t off = qh * a.D + d;                      // [seq][heads][D]
    if (a.o_dtype == MVLM_F32)
        *reinterpret_cast<f32x4*>((float*)a.O + off) = o * inv;
    else
        *reinterpret_cast<u32x2*>((uint16_t*)a.O + off) =
            u32x2{pack_f16x2(o[0] * inv, o[1] * inv), pack_f16x2(o[2] * inv, o[3] * inv)};
}

template <int KS, int DT, int NW>
static hipError_t launch_variant(hipStream_t s, const AttnArgs& a) {
    auto kernel = attention_kernel<KS, DT, NW>;
    constexpr int lds = NW * AttnLayout<KS, DT>::REGION;
    static_assert(lds <= ATTN_LDS_MAX, "attention LDS over budget");
    if (const hipError_t e = allow_dynamic_lds<attention_kernel<KS, DT, NW>>(ATTN_LDS_MAX); e != hipSuccess) return e;
    const dim3 grid((unsigned)((a.seq_q + 31) / 32), (unsigned)a.heads, (unsigned)a.splits);
    if (a.splits == 1) {
        launch_kernel(kernel, grid, dim3(64 * NW), (uint32_t)lds, s, a);
        return hipGetLastError();
    }
    launch_kernel_part(LaunchPart::First, kernel, grid, dim3(64 * NW), (uint32_t)lds, s, a);
    const int64_t items = (int64_t)a.seq_q * a.heads * (a.D / 4);
    launch_kernel_part(LaunchPart::Last, attention_combine_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256),
                       0, s, a);
    return hipGetLastError();
}

// Splits over keys: none when the (32-query tile, head) blocks alone cover the
// CUs or the keys are at most 48 tiles (1536 keys); otherwise enough for about
// two blocks per CU, keeping at least two key tiles per split.  The split path
// pays a second launch (~3-4 us): one 32-head decode block per head with 16
// waves measured 5.0 us against 9.3 us split at 512 keys, and 9.9 us against
// 10.6-11.1 us split at 2048.
// MVLM_ATTN_SPLITS=<n> forces the split count (tuning runs; read where the
// workspace is sized and at every launch, so set it before creating the op).
static int pick_splits(int seq_q, int seq_kv, int heads, int num_cus) {
    const int64_t blocks = (int64_t)(seq_q + 31) / 32 * heads;
    const int tiles = (seq_kv + 31) / 32;
    if (const char* force = std::getenv("MVLM_ATTN_SPLITS")) {
        const int f = std::atoi(force);
        if (f >= 1 && f <= 32 && f <= tiles) return f;
    }
    if (blocks >= num_cus || tiles <= 48) return 1;
    const int64_t want = (2 * (int64_t)num_cus + blocks - 1) / blocks;
    return (int)std::max<int64_t>(1, std::min<int64_t>({want, tiles / 2, 32}));
}

size_t attention_workspace_bytes(int seq_q, int seq_kv, int heads, int head_dim, int num_cus) {
    const int splits = pick_splits(seq_q, seq_kv, heads, num_cus);
    if (splits == 1) return 0;
    return (size_t)splits * seq_q * heads * (head_dim + 2) * sizeof(float);
}

// Waves per block: the fewest block rounds times key tiles per wave, with
// blocks per CU bounded by LDS and by the resident waves the register use
// allows (about 3 per SIMD up to 64 dims, 2 up to 96, 1 beyond); ties go to
// fewer waves.
template <int KS, int DT>
static int pick_waves(int blocks, int key_tiles, int num_cus) {
    constexpr int region = AttnLayout<KS, DT>::REGION;
    constexpr int waves_per_cu = DT <= 2 ? 12 : DT == 3 ? 8 : 4;
    int best = 1;
    int64_t best_cost = INT64_MAX;
    for (int nw = 1; nw <= 16; nw *= 2) {
        if (nw * region > ATTN_LDS_MAX) break;
        const int per_cu = std::max(1, std::min(ATTN_LDS_MAX / (nw * region), waves_per_cu / nw));
        const int64_t rounds = (blocks + (int64_t)num_cus * per_cu - 1) / ((int64_t)num_cus * per_cu);
        const int64_t cost = rounds * ((key_tiles + nw - 1) / nw);
        if (cost < best_cost) {
            best_cost = cost;
            best = nw;
        }
    }
    return best;
}

// MVLM_ATTN_WAVES=<1|2|4|8|16> forces the waves per block (tuning runs; read at
// every launch).
template <int KS, int DT>
static hipError_t launch_dims(hipStream_t s, const AttnArgs& a, int num_cus) {
    const int blocks = (a.seq_q + 31) / 32 * a.heads * a.splits;
    int nw = pick_waves<KS, DT>(blocks, a.tiles_per_split, num_cus);
    const char* force = std::getenv("MVLM_ATTN_WAVES");
    if (force) {
        const int f = std::atoi(force);
        if ((f == 1 || f == 2 || f == 4 || f == 8 || f == 16) && f * AttnLayout<KS, DT>::REGION <= ATTN_LDS_MAX) nw = f;
    }
    switch (nw) {
        case 1: return launch_variant<KS, DT, 1>(s, a);
        case 2: return launch_variant<KS, DT, 2>(s, a);
        case 4: return launch_variant<KS, DT, 4>(s, a);
        case 8: return launch_variant<KS, DT, 8>(s, a);
        default:
            if constexpr (16 * AttnLayout<KS, DT>::REGION <= ATTN_LDS_MAX) return launch_variant<KS, DT, 16>(s, a);
            return hipErrorInvalidValue;
    }
}

hipError_t launch_attention(hipStream_t s, const void* Q, const void* K, const void* V, void* O, int o_dtype,
                            int seq_q, int seq_kv, int heads, int head_dim, int causal, float scale, int num_cus,
                            void* workspace, size_t workspace_bytes) {
    AttnArgs a{};
    a.splits = pick_splits(seq_q, seq_kv, heads, num_cus);
    const int tiles = (seq_kv + 31) / 32;
    a.tiles_per_split = (tiles + a.splits - 1) / a.splits;
    a.ws = (float*)workspace;
    // the split count is re-chosen here; a workspace sized for fewer splits
    // (MVLM_ATTN_SPLITS changed after the op was made) is refused
    if (a.splits > 1 &&
        (!workspace || workspace_bytes < (size_t)a.splits * seq_q * heads * (head_dim + 2) * sizeof(float)))
        return hipErrorInvalidValue;
    a.Q = (const uint16_t*)Q; a.K = (const uint16_t*)K; a.V = (const uint16_t*)V; a.O = O;
    a.o_dtype = o_dtype;
    a.seq_q = seq_q; a.seq_kv = seq_kv; a.heads = heads; a.D = head_dim;
    a.causal = causal;
    a.scale_log2 = scale * 1.4426950408889634f;
    if (head_dim <= 32) return launch_dims<2, 1>(s, a, num_cus);
    if (head_dim <= 48) return launch_dims<3, 2>(s, a, num_cus);
    if (head_dim <= 64) return launch_dims<4, 2>(s, a, num_cus);
    if (head_dim <= 80) return launch_dims<5, 3>(s, a, num_cus);
    if (head_dim <= 96) return launch_dims<6, 3>(s, a, num_cus);
    if (head_dim <= 112) return launch_dims<7, 4>(s, a, num_cus);
    if (head_dim <= 128) return launch_dims<8, 4>(s, a, num_cus);
    return hipErrorInvalidValue;
}

}  // namespace mvlm
