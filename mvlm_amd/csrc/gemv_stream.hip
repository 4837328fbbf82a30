// Decode GEMV for every packed weight format, one or several independent
// problems per launch:  y_p[m][n] = sum_k x_p[m][k] * w_p(n, k), M = 1 (and,
// for quantized weights, M <= 4: batched decode, every weight chunk converted
// once and multiplied with the M rows of x).
//
// Replaces gemv (src/kernels/gemm.cl:215-270) and adds the dequantizing
// Q8_0 / Q4_0 GEMV the reference plans (README.md:57).  A decode GEMV is one
// pass over the weight, so the kernel is organised around having all of a
// wave's HBM requests in flight before any arithmetic, and around few, large
// launches (a dependent launch costs ~1.6 us on MI355X, the time to stream
// ~10 MB):
//
//  * a "chunk" is one 16-byte vector per lane, 1 KiB per wave, of one weight
//    row: 4 fp32, 8 fp16/bf16, 16 Q8_0 codes (half a block) or 32 Q4_0 codes
//    (one block) per lane;
//  * a wave owns R rows x CW consecutive chunks (R*CW = 4: one contiguous
//    4 KiB region when a row is CW chunks long) and issues every code load,
//    every scale load and the matching x loads back to back; only then does
//    it convert and accumulate;
//  * rows longer than CW chunks are split over SPLIT = 2 or 4 waves of a
//    block (wave w takes chunks [w*CW, (w+1)*CW)); partial sums meet in LDS;
//  * one launch serves up to MAX_GROUP independent problems of the same
//    weight format (e.g. Phi-1.5's QKV and fc1, which read the same input, or
//    its dense and fc2 projections); blocks are dealt to problems in order.
// Codes become fp32 in registers: v_cvt_f32_i32 with a byte select for
// Q8_0, masked nibbles through v_cvt_f32_ubyte* for Q4_0.  The block scale is
// applied once per half block (Q8_0) or block (Q4_0):
//   Q8_0: acc += d * sum_j x_j q_j
//   Q4_0: acc += d * (sum_j x_j c_j - 8 sum_j x_j),  c_j the 4-bit code.
// This is the GGUF dequantization (w = d*q, w = (c-8)*d) with d factored out
// of each block: different rounding, same value within the fp32 tolerance.
#include "gemv_common.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <vector>

namespace mvlm {

// ---- the kernel ------------------------------------------------------------

// One problem of a grouped launch.  Chunk c of a row covers bytes
// [1024c, 1024c + 1024) of the row, lane l the 16 bytes at 1024c + 16l, i.e.
// weights [WPL*(64c + l), WPL*(64c + l + 1)).  K % WPL == 0, so a lane's vector
// lies entirely below K or entirely above it; lanes above K load the row's
// first vector instead (always in bounds) and discard the result, which keeps
// every load unconditional and lets them all issue before the first wait.
struct StreamProblem {
    const void* x;                 // [M][K]
    const uint8_t* codes;
    const uint16_t* scales;
    void* y;                       // [M][N]
    int64_t ld_bytes;
    int N, K, y_dtype;
    int M;                         // rows of x (1 for MX = 1; 2 for MX = 2; 3..4 for MX = 4)
    int shape;                     // index into kShapes
    int rows_per_block;            // block j owns rows [j*rows_per_block, (j+1)*rows_per_block) below N
    int block_begin;               // first block of this problem in the grid
    int ep_on;
    int dep;                       // x is the output of the launch's attention (waits for it)
    int prod;                      // y holds the launch's attention's q, k, v (device-scope stores, flags)
    Epilogue ep;                   // applied to y when ep_on
};

constexpr int MAX_GROUP = 8;
#ifndef MVLM_STREAM_WAVES
#define MVLM_STREAM_WAVES 8
#endif
constexpr int NWAVE = MVLM_STREAM_WAVES;   // waves per block

// ---- decode attention carried by a grouped launch ----------------------------
//
// Decode attention: one new query per head against the KV cache (the work of
// attention_decode, src/kernels/attention.cl:197-295).  Phi-1.5 runs it
// between its grouped {QKV, fc1} and {dense, fc2} GEMVs; as a launch of its
// own it costs a kernel boundary for ~4 MB of cache reads.  A grouped launch
// can carry it instead, in one of two ways:
//  * before its readers (mode 0, mvlm_plan_add_attention): the attention's
//    workgroups come first in the {dense, fc2} launch; the workgroups of the
//    problems whose x is o issue their weight loads, wait (one lane polls)
//    until every head is done, then stage o in LDS;
//  * after its producer (mode 1, mvlm_plan_add_attention_decode_step): q and
//    the new key and value are the three thirds of one problem's output (the
//    fused QKV projection, moondream2.cpp:369-440 with the cache append of
//    :305-316, :419); the attention's workgroups follow that problem's in the
//    {QKV, fc1} launch, load their cached keys and values, wait for the
//    producer workgroups that write their head's rows, then append the new
//    key and value to the cache (fp16) and attend over cached + 1 keys.  The
//    next launch reads o after a kernel boundary.
// Attention workgroup (head h, key split s) runs an online softmax per wave,
// merges its waves in LDS and stores a partial result (unnormalised output,
// running max, sum of weights); the last split of a head to finish (a
// device-scope counter per head) merges the splits and writes o[h].
// Counters live in a sync area of the launch site (one per fused plan entry,
// zeroed once) and only ever grow, so no launch resets anything and no
// atomic is awaited by every waiting workgroup (a counter that 256
// workgroups bump serialises for ~3 us):
//   byte 0      u64  done (mode 0): heads finished over all launches; the
//                    bump that completes a launch's heads writes go
//   byte 256    u32  error word
//   byte 1024   u32  go[16] (mode 0), 128 bytes apart: launches completed;
//                    waiting workgroup c polls go[c % 16]
//   byte 4096   u64  head[h], 64 bytes apart: splits of head h finished; the
//                    bump reaching a multiple of splits merges
//   byte 16384  u32  seen[c] (mode 0): launches waiting workgroup c has waited
//                    through (its own word: it waits for go >= seen + 1)
//   byte 32768  u32  flag[j] (mode 1): launches producer workgroup j has
//                    finished (raised once its output stores are complete)
//   byte 49152  u32  aseen[b] (mode 1): launches attention workgroup b has
//                    waited through
// Launches of one site run one after another on the stream, so each
// launch's counts are whole multiples when the next begins.
// Only workgroups that wait (mode 0: the readers of o; mode 1: the attention)
// wait, and only on workgroups that never wait, so the launch completes as
// long as the waiting ones cannot fill the device by themselves (checked on
// the host against the kernel's occupancy).  A wait still gives up after
// 20 ms: the workgroup then stores NaN instead of its outputs and sets the
// error word (read by mvlm_plan_check, which then clears the area).
// Data crossing workgroups (producer rows, partials, o) moves with
// device-scope (sc1) stores and loads, and every such store is complete
// (s_waitcnt vmcnt(0)) before the counter or flag that publishes it.
constexpr int SYNC_DONE_B = 0, SYNC_ERR_B = (int)SYNC_ERR_OFFSET, SYNC_GO_B = 1024, SYNC_HEAD_B = 4096,
              SYNC_SEEN_B = 16384, SYNC_FLAG_B = 32768, SYNC_ASEEN_B = 49152;
constexpr int SYNC_GO_N = 16;
constexpr int ATTN_MAX_HEADS = (SYNC_SEEN_B - SYNC_HEAD_B) / 64;
constexpr int ATTN_MAX_CONSUMERS = (SYNC_FLAG_B - SYNC_SEEN_B) / 4;
constexpr int ATTN_MAX_PRODUCERS = (SYNC_ASEEN_B - SYNC_FLAG_B) / 4;
constexpr int ATTN_MAX_BLOCKS = ((int)SYNC_BYTES - SYNC_ASEEN_B) / 4;
static_assert(SYNC_BYTES == 65536, "sync area layout");
constexpr int ATTN_NL = 2;                     // key (and value) loads per lane and iteration
constexpr int ATTN_MAX_SPLITS = 32;
constexpr uint64_t ATTN_TIMEOUT = 2000000;     // s_memrealtime ticks (100 MHz): 20 ms

struct StreamAttn {
    const uint16_t* q;         // mode 0: fp16 [heads][D]
    const float* qkv;          // mode 1: fp32 [3][heads][D]: q, new key, new value
    uint16_t* k;               // fp16 caches [.][heads][D]: rows [0, cached) read; mode 1 writes row `cached`
    uint16_t* v;
    float* o;                  // [heads][D]
    float* part_o;             // [heads][splits][D] unnormalised outputs of the splits
    float* part_ml;            // [heads][splits][2] running max (exp2 domain) and sum of weights
    uint8_t* sync;             // the site's sync area (merge != 0)
    int heads, D;
    int cached;                // keys read from the cache
    int seq_kv;                // keys attended: cached (mode 0), cached + 1 (mode 1)
    int splits, keys_per_split, blocks;
    int first;                 // grid index of the first attention workgroup
    int mode;                  // 0: before the problems reading o; 1: after the problem writing qkv
    int step;                  // q, the new key and value from qkv, appended to the caches
    int merge;                 // the last split merges (else attn_merge_kernel does)
    int consumers;             // mode 0: workgroups that wait for o
    int prod_rpb, prod_blocks; // mode 1: the producer problem's rows per workgroup and workgroups (first in the grid)
    float scale_log2;          // scale * log2(e)
    uint32_t wait_ticks;       // bound of every wait, s_memrealtime ticks (ATTN_TIMEOUT)
};

struct StreamGroup {
    StreamProblem p[MAX_GROUP];
    int count;
    StreamAttn at;             // used by the launches that carry attention
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}
__device__ __forceinline__ void stores_complete() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
template <typename T>
__device__ __forceinline__ T* sync_word(const StreamAttn& a, int byte) {
    return reinterpret_cast<T*>(a.sync + byte);
}
__device__ __forceinline__ uint64_t sync_add64(uint64_t* p) {
    return __hip_atomic_fetch_add(p, (uint64_t)1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_store(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t sync_load(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// lane 0's value of a 64-bit counter result, in every lane
__device__ __forceinline__ uint64_t first_lane64(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
__device__ __forceinline__ float f16_round(float x) { return f16_bits_to_f32(f32_to_f16_bits(x)); }

// Head h's o is stored and complete: count it; the count completing a
// launch's heads publishes the launch number in every go line (mode 0).
__device__ __forceinline__ void attn_head_done(const StreamAttn& a, int lane) {
    if (a.mode != 0) return;
    uint64_t old = 0;
    if (lane == 0) old = sync_add64(sync_word<uint64_t>(a, SYNC_DONE_B));
    const uint64_t n = first_lane64(old) + 1;
    if (n % (uint64_t)a.heads == 0 && lane < SYNC_GO_N)
        sync_store(sync_word<uint32_t>(a, SYNC_GO_B + 128 * lane), (uint32_t)(n / (uint64_t)a.heads));
}

// Mode 1, attention workgroup b of head h: wait until every producer
// workgroup writing rows [h D, h D + D) of each third of qkv has raised its
// flag to aseen[b] + 1, and count the launch in aseen[b].  False when the
// wait gave up.
__device__ __forceinline__ bool attn_wait_producers(const StreamAttn& a, int b, int h, int wave, int lane,
                                                    uint32_t* flag_ok) {
    if (wave == 0) {
        uint32_t* aseen = sync_word<uint32_t>(a, SYNC_ASEEN_B + 4 * b);
        const uint32_t want = __builtin_amdgcn_readfirstlane(sync_load(aseen)) + 1;
        const uint32_t* flags = sync_word<uint32_t>(a, SYNC_FLAG_B);
        const int per = (a.D - 1) / a.prod_rpb + 2;   // workgroups a range of D rows can touch
        bool ok = true;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (true) {
            bool up = true;
            for (int i = lane; i < 3 * per; i += 64) {
                const int third = i / per, t = i - third * per;
                const int r0 = third * a.heads * a.D + h * a.D;
                const int j = r0 / a.prod_rpb + t;
                if (j <= (r0 + a.D - 1) / a.prod_rpb) up &= (int32_t)(sync_load(flags + j) - want) >= 0;
            }
            if (__builtin_amdgcn_ballot_w64(!up) == 0) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 > (uint64_t)a.wait_ticks) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (lane == 0) {
            sync_store(aseen, want);
            if (!ok) sync_store(sync_word<uint32_t>(a, SYNC_ERR_B), 1u);
            *flag_ok = ok ? 1u : 0u;
        }
    }
    lds_barrier();
    return *flag_ok != 0;
}

// A producer workgroup (mode 1) has stored its rows with device-scope stores:
// once every wave's stores are complete, raise its flag.
__device__ __forceinline__ void attn_producer_done(const StreamAttn& a, int j, int wave, int lane) {
    stores_complete();
    lds_barrier();
    if (wave == 0 && lane == 0) {
        uint32_t* flag = sync_word<uint32_t>(a, SYNC_FLAG_B + 4 * j);
        sync_store(flag, sync_load(flag) + 1);   // its own word: no other writer
    }
}

// One attention workgroup b: keys [k0, k1) of head h.  Wave w takes keys
// k0 + 16w + 128i .. (D = 64; 8 lanes of 16 bytes per key, ATTN_NL keys per
// lane and iteration), scores in the exp2 domain.  In mode 1 the split that
// holds key `cached` takes the new key from qkv (wave 0) and writes it and
// the new value to the caches.  flag_ok: one word of LDS for the wait.
template <int D>
__device__ __forceinline__ void attn_decode_block(const StreamAttn& a, int b, float* lds, uint32_t* flag_ok, int wave,
                                                  int lane) {
    constexpr int LPK = D / 8;                 // lanes per key
    constexpr int KPI = 64 / LPK;              // keys per wave-wide load
    constexpr int KPW = ATTN_NL * KPI;         // keys per wave and iteration
    constexpr int DPL = D / 64;                // output dims per lane in the merges
    const int h = b / a.splits, sp = b - h * a.splits;
    // a step's last split holds only the new key (index `cached`); the others
    // cut the cached keys
    const bool new_key = a.step && sp == a.splits - 1;
    const int k0 = sp * a.keys_per_split, kc1 = new_key ? k0 : min(k0 + a.keys_per_split, a.cached);
    const int sub = lane % LPK, kl = lane / LPK;
    const int64_t key_stride = (int64_t)a.heads * D;
    const int col = h * D + sub * 8;
    bool ok = true;
    float qf[8];
    float m = -INFINITY, l = 0.0f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;
    // online softmax over N keys of the wave (one per lane group): packed fp16
    // key and value rows of this lane's 8 dims; keys with valid false score -inf
    auto process = [&](const u32x4* kp, const u32x4* vp, const bool* valid, auto n_keys) {
        constexpr int N = decltype(n_keys)::value;
        float s[N], mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                d = __builtin_fmaf(qf[2 * e], f16_bits_to_f32((uint16_t)(kp[j][e] & 0xFFFFu)), d);
                d = __builtin_fmaf(qf[2 * e + 1], f16_bits_to_f32((uint16_t)(kp[j][e] >> 16)), d);
            }
#pragma unroll
            for (int off = 1; off < LPK; off <<= 1) d += __shfl_xor(d, off);
            s[j] = valid[j] ? d : -INFINITY;
            mx = fmaxf(mx, s[j]);
        }
#pragma unroll
        for (int off = LPK; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        const float mn = fmaxf(m, mx);               // finite: the first key of the group is real
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= alpha;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const float p = __builtin_amdgcn_exp2f(s[j] - mn);
            l += p;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                o[2 * e] = __builtin_fmaf(p, f16_bits_to_f32((uint16_t)(vp[j][e] & 0xFFFFu)), o[2 * e]);
                o[2 * e + 1] = __builtin_fmaf(p, f16_bits_to_f32((uint16_t)(vp[j][e] >> 16)), o[2 * e + 1]);
            }
        }
        m = mn;
    };
    // q, rounded to fp16, in the exp2 domain: from qkv (a step, after its
    // producers in mode 1) or the fp16 q
    auto load_q = [&]() {
        if (a.step) {
            if (a.mode == 1 && a.prod_blocks > 0) ok = attn_wait_producers(a, b, h, wave, lane, flag_ok);
            const __amdgpu_buffer_rsrc_t qr = dev_rsrc(a.qkv, 3 * a.heads * D * 4);
            const u32x4 u0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, col * 4, 0, kCpolDevice));
            const u32x4 u1 =
                __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, col * 4 + 16, 0, kCpolDevice));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                qf[e] = f16_round(__uint_as_float(u0[e])) * a.scale_log2;
                qf[4 + e] = f16_round(__uint_as_float(u1[e])) * a.scale_log2;
            }
        } else {
            const u32x4 u = *reinterpret_cast<const u32x4*>(a.q + col);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qf[2 * j] = f16_bits_to_f32((uint16_t)(u[j] & 0xFFFFu)) * a.scale_log2;
                qf[2 * j + 1] = f16_bits_to_f32((uint16_t)(u[j] >> 16)) * a.scale_log2;
            }
        }
    };
    // the first iteration's cached keys and values, requested before q (they
    // do not depend on the producers)
    // (through buffer descriptors: 32-bit offsets, the caches being checked
    // below 2 GiB on the host)
    u32x4 kr[ATTN_NL], vr[ATTN_NL];
    int base = k0 + wave * KPW;
    const int cache_bytes = (int)((int64_t)(a.cached + 1) * key_stride * 2);
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(a.k, 0, cache_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(a.v, 0, cache_bytes, 0x00020000);
    auto load_kv = [&](int at) {
#pragma unroll
        for (int j = 0; j < ATTN_NL; ++j) {
            const int r = min(at + j * KPI + kl, kc1 - 1);
            kr[j] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, (int)((r * key_stride + col) * 2), 0, 2));
        }
#pragma unroll
        for (int j = 0; j < ATTN_NL; ++j) {
            const int r = min(at + j * KPI + kl, kc1 - 1);
            vr[j] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, (int)((r * key_stride + col) * 2), 0, 2));
        }
    };
    if (base < kc1) load_kv(base);
    load_q();
    if (new_key) {
        if (wave == 0) {   // the new key and value, rounded to fp16: attended and appended to the caches
            const __amdgpu_buffer_rsrc_t qr = dev_rsrc(a.qkv, 3 * a.heads * D * 4);
            u32x4 kb[1], vb[1];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int off = col * 4 + 16 * half;
                const u32x4 kf = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                               qr, a.heads * D * 4 + off, 0, kCpolDevice));
                const u32x4 vf = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                               qr, 2 * a.heads * D * 4 + off, 0, kCpolDevice));
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    kb[0][2 * half + e] = (uint32_t)f32_to_f16_bits(__uint_as_float(kf[2 * e])) |
                                          ((uint32_t)f32_to_f16_bits(__uint_as_float(kf[2 * e + 1])) << 16);
                    vb[0][2 * half + e] = (uint32_t)f32_to_f16_bits(__uint_as_float(vf[2 * e])) |
                                          ((uint32_t)f32_to_f16_bits(__uint_as_float(vf[2 * e + 1])) << 16);
                }
            }
            const bool valid[1] = {kl == 0};
            process(kb, vb, valid, std::integral_constant<int, 1>{});
            if (kl == 0) {   // row `cached` of head h, this lane's 8 dims
                *reinterpret_cast<u32x4*>(a.k + (int64_t)a.cached * key_stride + col) = kb[0];
                *reinterpret_cast<u32x4*>(a.v + (int64_t)a.cached * key_stride + col) = vb[0];
            }
        }
    } else {
        for (; base < kc1; base += NWAVE * KPW) {
            bool valid[ATTN_NL];
#pragma unroll
            for (int j = 0; j < ATTN_NL; ++j) valid[j] = base + j * KPI + kl < kc1;
            process(kr, vr, valid, std::integral_constant<int, ATTN_NL>{});
            if (base + NWAVE * KPW < kc1) load_kv(base + NWAVE * KPW);
        }
    }
    // sums over the wave's key groups: lanes of one sub end with the wave's totals
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) {
        l += __shfl_xor(l, off);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += __shfl_xor(o[e], off);
    }
    float* mine = lds + wave * (D + 2);
    if (lane < LPK) {
#pragma unroll
        for (int e = 0; e < 8; ++e) mine[lane * 8 + e] = o[e];
    }
    if (lane == 0) {
        mine[D] = m;
        mine[D + 1] = l;
    }
    __syncthreads();
    if (wave != 0) return;
    // merge the waves (a wave without keys has m = -inf: weight 0); lane owns
    // dims lane + 64 t
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, lds[w * (D + 2) + D]);
    float L = 0.0f, acc[DPL];
#pragma unroll
    for (int t = 0; t < DPL; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
        const float f = __builtin_amdgcn_exp2f(lds[w * (D + 2) + D] - M);
        L = __builtin_fmaf(lds[w * (D + 2) + D + 1], f, L);
#pragma unroll
        for (int t = 0; t < DPL; ++t) acc[t] = __builtin_fmaf(lds[w * (D + 2) + lane + 64 * t], f, acc[t]);
    }
    if (!ok) {   // a wait gave up: NaN out
        M = __builtin_nanf("");
#pragma unroll
        for (int t = 0; t < DPL; ++t) acc[t] = M;
    }
    const __amdgpu_buffer_rsrc_t orr = dev_rsrc(a.o + h * D, D * 4);
    if (a.splits == 1) {
#pragma unroll
        for (int t = 0; t < DPL; ++t)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc[t] / L), orr, (lane + 64 * t) * 4, 0,
                                                 kCpolDevice);
        stores_complete();
        attn_head_done(a, lane);
        return;
    }
    const __amdgpu_buffer_rsrc_t por = dev_rsrc(a.part_o + (int64_t)h * a.splits * D, a.splits * D * 4);
    const __amdgpu_buffer_rsrc_t pmr = dev_rsrc(a.part_ml + (int64_t)h * a.splits * 2, a.splits * 8);
#pragma unroll
    for (int t = 0; t < DPL; ++t)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc[t]), por, (sp * D + lane + 64 * t) * 4,
                                             0, kCpolDevice);
    if (lane == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, M), pmr, sp * 8, 0, kCpolDevice);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, L), pmr, sp * 8 + 4, 0, kCpolDevice);
    }
    if (!a.merge) return;   // attn_merge_kernel combines the splits
    stores_complete();
    uint64_t arrived = 0;
    if (lane == 0) arrived = sync_add64(sync_word<uint64_t>(a, SYNC_HEAD_B + 64 * h));
    if ((first_lane64(arrived) + 1) % (uint64_t)a.splits != 0) return;
    // the last split of head h merges all of them.  Lane s < splits reads
    // split s's max and sum; the outputs come in as 16-byte pieces, 256
    // floats per wave-wide load (lane j: dims 4j % D .. + 3 of split
    // (256 i + 4 j) / D), four loads at a time, loads past the splits
    // reading zeros.
    constexpr int NB = 4;
    const int ni = (a.splits * D + 255) / 256;
    u32x4 pv[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
        pv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(por, (256 * i + 4 * lane) * 4, 0,
                                                                               kCpolDevice));
    const float ms = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pmr, lane * 8, 0, kCpolDevice));
    const float ls = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pmr, lane * 8 + 4, 0, kCpolDevice));
    float Mh = lane < a.splits ? ms : -INFINITY;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) Mh = fmaxf(Mh, __shfl_xor(Mh, off));
    const float fs = lane < a.splits ? __builtin_amdgcn_exp2f(ms - Mh) : 0.0f;
    float Lh = lane < a.splits ? ls * fs : 0.0f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) Lh += __shfl_xor(Lh, off);
    float r4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i0 = 0; i0 < ni; i0 += NB) {
        if (i0 > 0) {
#pragma unroll
            for (int i = 0; i < NB; ++i)
                pv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      por, (256 * (i0 + i) + 4 * lane) * 4, 0, kCpolDevice));
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int split = min((256 * (i0 + i) + 4 * lane) / D, ATTN_MAX_SPLITS - 1);   // zeros past the splits
            const float f = __shfl(fs, split);
#pragma unroll
            for (int e = 0; e < 4; ++e) r4[e] = __builtin_fmaf(__uint_as_float(pv[i][e]), f, r4[e]);
        }
    }
    // lanes holding the same dims: j, j + D/4, ... (D = 64: 4 of them, D = 128: 2)
#pragma unroll
    for (int off = D / 4; off < 64; off <<= 1)
#pragma unroll
        for (int e = 0; e < 4; ++e) r4[e] += __shfl_xor(r4[e], off);
    if (lane < D / 4) {
        u32x4 out;
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = __builtin_bit_cast(uint32_t, r4[e] / Lh);
        __builtin_amdgcn_raw_buffer_store_b128(out, orr, lane * 16, 0, kCpolDevice);
    }
    stores_complete();
    attn_head_done(a, lane);
}


// Mode 0, waiting workgroup c (of the launch's consumers): wait until this
// launch's heads are all done, i.e. go >= seen[c] + 1, and count the launch
// in seen[c] (lane 0 of wave 0).  Returns false when the wait gave up (the
// workgroup then stores NaN).
__device__ __forceinline__ bool attn_wait(const StreamAttn& a, int wave, int lane, uint32_t* flag) {
    if (wave == 0 && lane == 0) {
        const int c = (int)blockIdx.x - (int)gridDim.x + a.consumers;
        uint32_t* seen = sync_word<uint32_t>(a, SYNC_SEEN_B + 4 * c);
        const uint32_t want = sync_load(seen) + 1;
        const uint32_t* go = sync_word<uint32_t>(a, SYNC_GO_B + 128 * (c % SYNC_GO_N));
        uint32_t ok = 1;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while ((int32_t)(sync_load(go) - want) < 0) {
            if (__builtin_amdgcn_s_memrealtime() - t0 > (uint64_t)a.wait_ticks) {
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        sync_store(seen, want);
        if (!ok) sync_store(sync_word<uint32_t>(a, SYNC_ERR_B), 1u);
        *flag = ok;
    }
    lds_barrier();
    return *flag != 0;
}

// A decode attention on its own: its workgroups only (no wait), partials to
// the workspace, then attn_merge_kernel.
template <int D>
__global__ __launch_bounds__(64 * NWAVE) void attn_split_kernel(const StreamAttn a) {
    __shared__ float lds[NWAVE * (D + 2)];
    __shared__ uint32_t flag_ok;
    attn_decode_block<D>(a, (int)blockIdx.x, lds, &flag_ok, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
                         threadIdx.x & 63);
}

// o[h] from head h's split partials: one wave per head, lane d owns dims d + 64 t.
template <int D>
__global__ __launch_bounds__(64) void attn_merge_kernel(const StreamAttn a) {
    const int h = blockIdx.x, lane = threadIdx.x, S = a.splits;
    const float* ml = a.part_ml + (int64_t)h * S * 2;
    const float* po = a.part_o + (int64_t)h * S * D;
    float M = -INFINITY;
    for (int s = 0; s < S; ++s) M = fmaxf(M, ml[2 * s]);
    float L = 0.0f, acc[D / 64];
#pragma unroll
    for (int t = 0; t < D / 64; ++t) acc[t] = 0.0f;
    for (int s = 0; s < S; ++s) {
        const float f = __builtin_amdgcn_exp2f(ml[2 * s] - M);
        L = __builtin_fmaf(ml[2 * s + 1], f, L);
#pragma unroll
        for (int t = 0; t < D / 64; ++t) acc[t] = __builtin_fmaf(po[s * D + lane + 64 * t], f, acc[t]);
    }
#pragma unroll
    for (int t = 0; t < D / 64; ++t) a.o[h * D + lane + 64 * t] = acc[t] / L;
}

// Work shape of one wave by row length in 1 KiB chunks: R rows x CW chunks,
// the row split over SPLIT waves when it is longer than CW chunks.  A wave
// keeps 4 to 8 loads of 16 bytes per lane in flight; whole rows per wave
// (SPLIT = 1) need no combine step.  The first kByLength shapes are chosen by
// row length; the last is shape 3 with two rows per wave, used with 2..4 rows
// of x (each wave then stages half as many x bytes per code byte; with one
// row of x it measured slower).
struct Shape { int max_chunks, R, CW, SPLIT; };
constexpr Shape kShapes[] = {{1, 4, 1, 1}, {2, 2, 2, 1}, {4, 1, 4, 1}, {8, 1, 4, 2}, {16, 1, 8, 2}, {8, 2, 4, 2},
                             {2, 1, 2, 1}};
constexpr int kNumShapes = 7, kByLength = 5, kBatchLong = 5, kFewRows2 = 6;
// Shapes a problem that waits for the launch's attention (or writes its q, k
// and v) may take: rows of at most 4 KiB in HBM (with longer rows the
// registers holding the code loads push the kernel past its register budget).
constexpr bool kDepShape[] = {true, true, true, false, false, false, true};
static_assert(sizeof(kShapes) / sizeof(kShapes[0]) == kNumShapes, "one kernel case per shape");

// The rows [row0, row0 + R) of one wave (those below the block's end rb1),
// its chunks wsub*CW ... of each, against MX rows of x (vector m staged at
// LDS byte m * x_stride; rows of x at or past M repeat row M-1 and are not
// stored).  x and the scales are already being staged into LDS (staging loads
// were issued before these and complete first).
// ROLE 1 (a problem reading the launch's attention output): x is not staged
// yet; the wave waits for the attention after issuing its code loads, then
// stages x.  y_device: y (fp32) goes out with device-scope stores (the
// producer of the launch's attention's q, k, v).
template <class F, typename XT, int MX, int R, int CW, int SPLIT, int ROLE>
__device__ __forceinline__ void stream_rows(const StreamProblem& P, int rb0, int rb1, int64_t s_base, int x_stride,
                                            int x_region, uint8_t* lds, float (*part)[4 * MX], int wave,
                                            int lane, const StreamAttn& at, uint32_t* wait_ok, bool y_device) {
    constexpr int WPL = F::WPL;
    constexpr int XB = WPL * (int)sizeof(XT);        // x bytes per lane per chunk
    constexpr int SL = XB >= 16 ? XB / 16 : 1;       // 16-byte LDS slots per lane per chunk
    const int K = P.K, nb = K >> 5;
    const int wsub = wave % SPLIT;
    const int row0 = rb0 + (wave / SPLIT) * R;
    const bool active = row0 < rb1;

    // the codes: every load of this wave before any arithmetic, through a
    // buffer descriptor (32-bit offsets: the host keeps a weight's codes below
    // 4 GiB on this path)
    const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(P.codes), 0, (int)min((int64_t)P.N * P.ld_bytes, (int64_t)0x7FFFFFFF), 0x00020000);
    uint32_t rowo[R];
    int srow[R];                                      // row's scale byte offset in the staged region
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = (int64_t)min(row0 + r, rb1 - 1);
        rowo[r] = (uint32_t)(row * P.ld_bytes);
        srow[r] = (int)(row * (nb * 2) - s_base);
    }
    // The epilogue operands of the output this lane stores (lane j < R MX
    // stores output j), requested before the codes: the store at the end then
    // takes them from registers instead of waiting for a round trip to memory.
    constexpr int NV = R * MX;
    const int jr = (lane & (NV - 1)) / MX, jm = (lane & (NV - 1)) % MX;
    float eb = 0.0f, em = 1.0f, er = 0.0f;
    if (P.ep_on) {
        const int erow = min(row0 + jr, rb1 - 1);
        const int64_t eidx = MX == 1 ? (int64_t)erow : (int64_t)min(jm, P.M - 1) * P.N + erow;
        if (P.ep.bias) eb = load_as_f32(P.ep.bias, erow, P.ep.dtype);
        if (P.ep.mul) em = load_as_f32(P.ep.mul, eidx, P.ep.dtype);
        if (P.ep.res) er = load_as_f32(P.ep.res, eidx, P.ep.dtype);
    }
    u32x4 q[R][CW];
    int kk[CW];
    bool valid[CW];
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        const int c = wsub * CW + i;
        const int k = (64 * c + lane) * WPL;
        valid[i] = active && k < K;
        kk[i] = k < K ? k : 0;
#pragma unroll
        for (int r = 0; r < R; ++r)
            q[r][i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(cr, (int)(rowo[r] + (uint32_t)(kk[i] * 16 / WPL)), 0, 2));
    }
    __builtin_amdgcn_sched_barrier(0);

    // LDS byte offsets of this lane's x slots.  A valid lane's slice of chunk c
    // starts at slot (64c + lane) * SL, and x_slot moves its slot v to
    // v ^ xt with xt = ((lane * SL) >> 4) & (SL - 1) for every c; a lane past K
    // reads the first slots instead (any in-bounds bytes: its result is
    // discarded).  So one add per read: xbase[i] + xoff[v].
    int xbase[CW], xoff[SL];
#pragma unroll
    for (int i = 0; i < CW; ++i) xbase[i] = valid[i] ? (64 * (wsub * CW + i) + lane) * SL * 16 : 0;
    {
        const int xt = ((lane * SL) >> 4) & (SL - 1);
#pragma unroll
        for (int v = 0; v < SL; ++v) xoff[v] = (v ^ xt) << 4;
    }

    // staging done for every wave -> x and scales from LDS, chunk by chunk
    bool ok = true;
    if constexpr (ROLE == 1) {
        ok = attn_wait(at, wave, lane, wait_ok);
        stage_to_lds<(XB >= 16 ? 16 : 4), SL, NWAVE, kCpolDevice>(lds, (const uint8_t*)P.x, K * (int)sizeof(XT),
                                                                    wave, lane);
        wait_vmcnt<0>();
    } else {
        wait_vmcnt<R * CW>();
    }
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // Q4_0: the block sums of each row of x (the -8 offset's term, sxl[m][b]),
    // once per workgroup into LDS after the scales, instead of once per chunk,
    // row and wave
    constexpr bool kSumX = std::is_same_v<F, Q4Fmt>;
    const float* sxl = reinterpret_cast<const float*>(lds + x_region + ((P.rows_per_block * nb * 2 + 30 + 1023) & ~1023));
    if constexpr (kSumX) {
        for (int t = threadIdx.x; t < MX * nb; t += 64 * NWAVE) {
            const int m = MX == 1 ? 0 : t / nb, b = MX == 1 ? t : t - m * nb;
            const u32x4* xm = reinterpret_cast<const u32x4*>(lds + m * x_stride);
            XRaw<XT, WPL> xr;
#pragma unroll
            for (int v = 0; v < SL; ++v) {
                const u32x4 u = xm[x_slot<SL>(SL * b + v)];
                xr.d[4 * v + 0] = u[0]; xr.d[4 * v + 1] = u[1];
                xr.d[4 * v + 2] = u[2]; xr.d[4 * v + 3] = u[3];
            }
            const_cast<float*>(sxl)[t] = x_block_sum(xr);
        }
        // LDS-only fences around the barrier: the code loads stay in flight
        // (a full __syncthreads() would wait for them)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    float acc[R][MX];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MX; ++m) acc[r][m] = 0.0f;
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        if constexpr (MX == 1) {   // one row of x: the x slice is read once per chunk
            XRaw<XT, WPL> xr;
            const int xbyte = kk[i] * (int)sizeof(XT);
            if constexpr (XB >= 16) {
#pragma unroll
                for (int v = 0; v < SL; ++v) {
                    const u32x4 u = *reinterpret_cast<const u32x4*>(lds + xbase[i] + xoff[v]);
                    xr.d[4 * v + 0] = u[0]; xr.d[4 * v + 1] = u[1];
                    xr.d[4 * v + 2] = u[2]; xr.d[4 * v + 3] = u[3];
                }
            } else {   // XB == 8
                const u32x2 u = *reinterpret_cast<const u32x2*>(lds + xbyte);
                xr.d[0] = u[0]; xr.d[1] = u[1];
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint16_t dh = 0;
                if constexpr (F::QUANT)
                    dh = *reinterpret_cast<const uint16_t*>(lds + x_region + srow[r] + (kk[i] >> 5) * 2);
                float v;
                if constexpr (kSumX) v = chunk_dot_q4(q[r][i], dh, xr, sxl[kk[i] >> 5], acc[r][0]);
                else v = chunk_dot(F{}, q[r][i], dh, xr, acc[r][0]);
                acc[r][0] = valid[i] ? v : acc[r][0];
            }
            continue;
        }
#pragma unroll
        for (int m = 0; m < MX; ++m) {
            XRaw<XT, WPL> xr;
            const uint8_t* xl = lds + m * x_stride;
            const int xbyte = kk[i] * (int)sizeof(XT);
            if constexpr (XB >= 16) {
#pragma unroll
                for (int v = 0; v < SL; ++v) {
                    const u32x4 u = *reinterpret_cast<const u32x4*>(xl + xbase[i] + xoff[v]);
                    xr.d[4 * v + 0] = u[0]; xr.d[4 * v + 1] = u[1];
                    xr.d[4 * v + 2] = u[2]; xr.d[4 * v + 3] = u[3];
                }
            } else {   // XB == 8
                const u32x2 u = *reinterpret_cast<const u32x2*>(xl + xbyte);
                xr.d[0] = u[0]; xr.d[1] = u[1];
            }
            float sx = 0.0f;
            if constexpr (kSumX) sx = sxl[m * nb + (kk[i] >> 5)];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint16_t dh = 0;
                if constexpr (F::QUANT)
                    dh = *reinterpret_cast<const uint16_t*>(lds + x_region + srow[r] + (kk[i] >> 5) * 2);
                float v;
                if constexpr (kSumX) v = chunk_dot_q4(q[r][i], dh, xr, sx, acc[r][m]);
                else v = chunk_dot(F{}, q[r][i], dh, xr, acc[r][m]);
                acc[r][m] = valid[i] ? v : acc[r][m];
            }
        }
    }
    // the R x MX sums over the wave: lane j < R * MX ends with sum j = r * MX + m
    float flat[NV];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MX; ++m) flat[r * MX + m] = acc[r][m];
    const float tot = wave_sum_lanes<NV>(flat, lane);

    // y[m][row] with the epilogue (apply_epilogue's steps in its order, on the
    // operands loaded above), the NV outputs of a wave stored by NV lanes at once
    auto epilogue = [&](float v) {
        if (P.ep.bias) v += eb;
        if (P.ep.act == 1) v = gelu_tanh(v);
        else if (P.ep.act == 2) v = silu(v);
        if (P.ep.mul) v *= em;
        if (P.ep.res) v += er;
        return v;
    };
    auto store_row = [&](int row, int m, float v) {
        if constexpr (ROLE == 1) v = ok ? v : __builtin_nanf("");
        if (P.ep_on) v = epilogue(v);
        if (MX == 1 && y_device) {   // fp32 y (checked on the host), read by other workgroups of the launch
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), dev_rsrc(P.y, P.N * 4), row * 4, 0, kCpolDevice);
        } else if constexpr (MX == 1) {
            store_out(P.y, row, v, P.y_dtype);
        } else {
            store_out(P.y, (int64_t)m * P.N + row, v, P.y_dtype);
        }
    };
    if constexpr (SPLIT == 1) {
        if (lane < NV && active && row0 + jr < rb1 && (MX == 1 || jm < P.M)) store_row(row0 + jr, jm, tot);
    } else {
        if (lane < NV) part[wave][lane] = tot;
        __syncthreads();
        if (wsub == 0 && lane < NV && active) {
            float v = part[wave][lane];
#pragma unroll
            for (int s = 1; s < SPLIT; ++s) v += part[wave + s][lane];
            if (row0 + jr < rb1 && (MX == 1 || jm < P.M)) store_row(row0 + jr, jm, v);
        }
    }
}

// A block of NWAVE waves owns a contiguous range of at most R * NWAVE / SPLIT
// rows of one problem.
// Per block, x and the rows' block scales are staged in LDS once (direct
// global->LDS loads), so each x element crosses the L2->CU path once per
// block rather than once per wave; the weight codes go straight to
// registers.  Issue order: x and scale staging, then every code load, then
// the wait for the staging alone (vmcnt counts in issue order), the block
// barrier, the LDS reads, and the wait for the codes.
// ATTN: workgroups [at.first, at.first + at.blocks) compute the decode
// attention (attn_decode_block); the problems marked dep read its output as
// x, the problem marked prod writes its q, k and v.
template <class F, typename XT, int MX, bool ATTN>
__global__ __launch_bounds__(64 * NWAVE, MX == 1 ? F::MIN_WAVES : F::MIN_WAVES_BATCH) void gemv_stream_kernel(
    const StreamGroup g) {
    constexpr int XB = F::WPL * (int)sizeof(XT);
    constexpr int SL = XB >= 16 ? XB / 16 : 1;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float part[NWAVE][4 * MX];
    __shared__ uint32_t wait_ok;

    // the wave index is uniform: keep it in a scalar register so the staging
    // loops and row offsets are scalar code
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if constexpr (ATTN) {
        const int b = (int)blockIdx.x - g.at.first;
        if (b >= 0 && b < g.at.blocks) {
            if (g.at.D == 64) attn_decode_block<64>(g.at, b, reinterpret_cast<float*>(lds), &wait_ok, wave, lane);
            else attn_decode_block<128>(g.at, b, reinterpret_cast<float*>(lds), &wait_ok, wave, lane);
            return;
        }
    }
    int pi = 0;
#pragma unroll
    for (int i = 1; i < MAX_GROUP; ++i)
        if (i < g.count && (int)blockIdx.x >= g.p[i].block_begin) pi = i;
    const StreamProblem& P = g.p[pi];
    const bool dep = ATTN && P.dep;
    const int N = P.N, K = P.K, nb = K >> 5;
    const int rb0 = ((int)blockIdx.x - P.block_begin) * P.rows_per_block;
    const int rb1 = min(rb0 + P.rows_per_block, N);

    // stage the MX rows of x (and the block's scales) in LDS
    // (x_bytes is a multiple of XB, so of 16 when XB >= 16)
    const int x_bytes = K * (int)sizeof(XT);
    const int x_stride = (x_bytes + 1023) & ~1023;
    const int x_region = MX * x_stride;
    if (!dep) {
#pragma unroll
        for (int m = 0; m < MX; ++m)
            stage_to_lds<(XB >= 16 ? 16 : 4), SL, NWAVE>(
                lds + m * x_stride, (const uint8_t*)P.x + (m == 0 ? 0 : (int64_t)min(m, P.M - 1) * x_bytes), x_bytes,
                wave, lane);
    }
    int64_t s_base = 0;                               // global byte offset of the first staged scale byte
    if constexpr (F::QUANT) {
        const int64_t s_begin = (int64_t)rb0 * (nb * 2);
        const int64_t s_end = (int64_t)rb1 * (nb * 2);
        s_base = s_begin & ~(int64_t)15;
        const int s_bytes = (int)((s_end - s_base + 15) & ~(int64_t)15);
        stage_to_lds<16, 1, NWAVE>(lds + x_region, (const uint8_t*)P.scales + s_base, s_bytes, wave, lane);
    }
    __builtin_amdgcn_sched_barrier(0);

    auto rows = [&](auto shape) {   // uniform over the block
        constexpr int si = decltype(shape)::value;
        constexpr Shape S = kShapes[si];
        if (ATTN && kDepShape[si] && dep)
            stream_rows<F, XT, MX, S.R, S.CW, S.SPLIT, ATTN ? 1 : 0>(P, rb0, rb1, s_base, x_stride, x_region, lds, part,
                                                                     wave, lane, g.at, &wait_ok, false);
        else
            stream_rows<F, XT, MX, S.R, S.CW, S.SPLIT, 0>(P, rb0, rb1, s_base, x_stride, x_region, lds, part, wave,
                                                          lane, g.at, &wait_ok, ATTN && P.prod);
    };
    switch (P.shape) {
        case 0: rows(std::integral_constant<int, 0>{}); break;
        case 1: rows(std::integral_constant<int, 1>{}); break;
        case 2: rows(std::integral_constant<int, 2>{}); break;
        case 3: rows(std::integral_constant<int, 3>{}); break;
        case 4: rows(std::integral_constant<int, 4>{}); break;
        case kFewRows2:
            if constexpr (MX == 1) rows(std::integral_constant<int, kFewRows2>{});
            break;
        case kBatchLong:
            if constexpr (MX > 1) rows(std::integral_constant<int, kBatchLong>{});
            break;
    }
    if constexpr (ATTN)
        if (P.prod) attn_producer_done(g.at, (int)blockIdx.x - P.block_begin, wave, lane);
}

// ---- launch configuration ----------------------------------------------------

static int weight_wpl(int dtype) {
    return dtype == MVLM_Q8_0 ? 16 : dtype == MVLM_Q4_0 ? 32 : 16 / (int)dtype_size(dtype);
}

// index into kShapes for this weight's row length and mx rows of x, -1 if
// rows are too long.  2-chunk rows with one row of x take one row per wave
// when two per wave would leave fewer workgroups than the device has CUs
// (num_cus > 0; num_cus == 0 keeps the by-length shape, whose LDS footprint
// bounds the one-row-per-wave variant's).
static int stream_shape(const mvlm_weight* w, int mx, int num_cus) {
    const int64_t chunks = (weight_row_bytes(w) + 1023) / 1024;
    for (int i = 0; i < kByLength; ++i)
        if (chunks <= kShapes[i].max_chunks) {
            if (mx > 1 && i == 3) return kBatchLong;
            if (mx == 1 && i == 1 && ((int64_t)w->N + 2 * NWAVE - 1) / (2 * NWAVE) < num_cus) return kFewRows2;
            return i;
        }
    return -1;
}

static int rows_per_block(int shape) { return kShapes[shape].R * (NWAVE / kShapes[shape].SPLIT); }

// LDS bytes of one block: x, then the block's scales plus the alignment
// slack of their start, each rounded to the 1 KiB pieces the staging writes.
// Scale reads reach up to 15 bytes past the scale array, which the weight
// allocation pads.
static size_t stream_lds_bytes(const mvlm_weight* w, int x_dtype, int shape, int mx = 1) {
    const size_t x_bytes = (size_t)w->K * dtype_size(x_dtype);
    size_t bytes = (size_t)mx * ((x_bytes + 1023) & ~(size_t)1023);
    if (is_quant(w->dtype))
        bytes += ((size_t)rows_per_block(shape) * (size_t)(w->K / 32) * 2 + 30 + 1023) & ~(size_t)1023;
    if (w->dtype == MVLM_Q4_0) bytes += (size_t)mx * (w->K / 32) * 4;   // block sums of each row of x
    return bytes;
}

constexpr size_t STREAM_LDS_MAX = 152 * 1024;

// Rows of x a launch's kernel carries: M = 2 has its own kernel (two fmas per
// converted weight), M = 3 and 4 share the four-row kernel (rows at or past M
// repeat row M - 1 and are not stored).
static int batch_mx(int M) { return M <= 1 ? 1 : M == 2 ? 2 : 4; }

bool stream_supported(const mvlm_weight* w, int M) {
    const int shape = stream_shape(w, M, 0);
    if (M > 1 && (M > 4 || !is_quant(w->dtype))) return false;
    return shape >= 0 && w->K % weight_wpl(w->dtype) == 0 &&
           w->bytes <= 0x7FFFFFFF &&   // 32-bit code offsets of the buffer loads
           stream_lds_bytes(w, MVLM_F32, shape, batch_mx(M)) <= STREAM_LDS_MAX;
}

int stream_max_group() { return MAX_GROUP; }

// Blocks per launch: each problem gets the fewest blocks whose row slots hold
// its rows.  (Spreading a problem over more, part-filled blocks to even out
// the bytes per CU was measured slower on MI355X: every block stages all of
// x, so x traffic grows with the block count, and part-filled blocks idle
// waves.  Computing block bounds by division, even once per block, also cost
// ~0.2 us per launch.)
// Block order: mode 0, the attention's workgroups, then the problems' (those
// that wait for it last); mode 1, the producer problem's, the attention's,
// then the other problems'.
static unsigned partition(StreamGroup& g) {
    unsigned begin = 0;
    g.at.consumers = 0;
    bool placed = g.at.blocks == 0;
    if (!placed && g.at.mode == 0) {
        g.at.first = 0;
        begin = (unsigned)g.at.blocks;
        placed = true;
    }
    for (int i = 0; i < g.count; ++i) {
        StreamProblem& p = g.p[i];
        p.rows_per_block = rows_per_block(p.shape);
        p.block_begin = (int)begin;
        const unsigned nblk = (unsigned)((p.N + p.rows_per_block - 1) / p.rows_per_block);
        begin += nblk;
        if (p.dep) g.at.consumers += (int)nblk;
        if (p.prod) {
            g.at.prod_rpb = p.rows_per_block;
            g.at.prod_blocks = (int)nblk;
        }
        if (!placed && p.prod) {
            g.at.first = (int)begin;
            begin += (unsigned)g.at.blocks;
            placed = true;
        }
    }
    return begin;
}

template <class F, typename XT, int MX = 1, bool ATTN = false>
static hipError_t launch_group(hipStream_t s, StreamGroup& g, size_t lds) {
    auto kernel = gemv_stream_kernel<F, XT, MX, ATTN>;
    if (const hipError_t e = allow_dynamic_lds<gemv_stream_kernel<F, XT, MX, ATTN>>((int)STREAM_LDS_MAX);
        e != hipSuccess)
        return e;
    const unsigned blocks = partition(g);
    launch_kernel(kernel, dim3(blocks), dim3(64 * NWAVE), (uint32_t)lds, s, g);
    return hipGetLastError();
}

template <class F>
static hipError_t launch_group_x(hipStream_t s, int x_dtype, StreamGroup& g, size_t lds) {
    switch (x_dtype) {
        case MVLM_F32: return launch_group<F, float>(s, g, lds);
        case MVLM_F16: return launch_group<F, __half>(s, g, lds);
        case MVLM_BF16: return launch_group<F, __hip_bfloat16>(s, g, lds);
        default: return hipErrorInvalidValue;
    }
}

// Key splits of a decode attention: enough workgroups to spread the cache
// reads over the device (heads * splits ~ CUs), each split a whole number of
// workgroup iterations (NWAVE waves x ATTN_NL loads x keys per load).
static void attn_split(int heads, int D, int seq_kv, int num_cus, int* splits, int* keys_per_split) {
    const int kb = NWAVE * ATTN_NL * (64 / (D / 8));
    int want = std::max(1, (num_cus + heads - 1) / heads);
    if (const char* e = std::getenv("MVLM_DECODE_SPLITS")) want = std::max(1, std::atoi(e));   // tuning override
    const int s = std::max(1, std::min(std::min((seq_kv + kb - 1) / kb, want), ATTN_MAX_SPLITS));
    const int k = ((seq_kv + s - 1) / s + kb - 1) / kb * kb;
    *keys_per_split = k;
    *splits = (seq_kv + k - 1) / k;
}

static int attn_seq(const StreamAttnDesc& d) { return d.cached + (d.step ? 1 : 0); }

// Splits of the cached keys (none for a step over an empty cache), plus a
// step's split for the new key.  Every split of cached keys holds at least
// one key.
static void attn_layout(int heads, int head_dim, int cached, int step, int num_cus, int* splits, int* kps) {
    *splits = 0;
    *kps = 1;
    if (cached > 0) attn_split(heads, head_dim, cached, num_cus, splits, kps);
    *splits += step ? 1 : 0;
}

size_t stream_attn_workspace_bytes(int heads, int head_dim, int cached, int step, int num_cus) {
    if (heads < 1 || (head_dim != 64 && head_dim != 128) || cached < 0 || cached + step < 1) return 0;
    int splits = 1, kps = 0;
    attn_layout(heads, head_dim, cached, step, num_cus > 0 ? num_cus : 256, &splits, &kps);
    return ((size_t)heads * splits * head_dim * 4 + 15) / 16 * 16 + (size_t)heads * splits * 8;
}

// The device-side description of attention `d` (no problems attached).
static bool attn_fill(StreamAttn& a, const StreamAttnDesc& d, int num_cus) {
    const int seq = attn_seq(d);
    if ((d.head_dim != 64 && d.head_dim != 128) || d.heads < 1 || d.heads > ATTN_MAX_HEADS || seq < 1 ||
        d.cached < 0 || !d.k || !d.v || !d.o || !d.workspace || (d.step ? !d.qkv : !d.q) || (d.mode == 1 && !d.step))
        return false;
    if ((int64_t)(d.cached + 1) * d.heads * d.head_dim * 2 > (int64_t)1 << 31) return false;
    a = StreamAttn{};
    a.q = (const uint16_t*)d.q;
    a.qkv = (const float*)d.qkv;
    a.k = (uint16_t*)d.k;
    a.v = (uint16_t*)d.v;
    a.o = d.o;
    a.sync = (uint8_t*)d.sync;
    a.heads = d.heads;
    a.D = d.head_dim;
    a.cached = d.cached;
    a.seq_kv = seq;
    a.mode = d.mode;
    a.step = d.step ? 1 : 0;
    attn_layout(d.heads, d.head_dim, d.cached, d.step, num_cus, &a.splits, &a.keys_per_split);
    a.part_o = (float*)d.workspace;
    a.part_ml = a.part_o + (size_t)d.heads * a.splits * d.head_dim;
    a.blocks = d.heads * a.splits;
    a.scale_log2 = d.scale * 1.4426950408889634f;
    // MVLM_ATTN_WAIT_TICKS shortens the bound (read at every launch; tests of
    // the give-up path set it to 0 so that a wait gives up at its first poll)
    a.wait_ticks = (uint32_t)ATTN_TIMEOUT;
    if (const char* e = std::getenv("MVLM_ATTN_WAIT_TICKS")) a.wait_ticks = (uint32_t)std::strtoul(e, nullptr, 10);
    return a.blocks <= ATTN_MAX_BLOCKS;
}

// Fills g.at and orders the problems for the mode: mode 0 moves the problems
// that read o to the end (dep); mode 1 moves the problem whose fp32 output is
// qkv (N = 3 heads D) to the front (prod).  False when the launch cannot
// carry the attention.
static bool attach_attention(StreamGroup& g, const StreamAttnDesc& d, int x_dtype, int M, int num_cus,
                             size_t& lds) {
    if (M != 1 || !d.sync || !attn_fill(g.at, d, num_cus)) return false;
    g.at.merge = 1;
    StreamProblem sorted[MAX_GROUP];
    int n = 0;
    if (d.mode == 0) {
        if (x_dtype != MVLM_F32) return false;
        for (int pass = 0; pass < 2; ++pass)
            for (int i = 0; i < g.count; ++i)
                if ((g.p[i].x == (const void*)d.o) == (pass == 1)) {
                    sorted[n] = g.p[i];
                    sorted[n++].dep = pass;
                }
        if (sorted[g.count - 1].dep == 0) return false;   // nothing reads o
        for (int i = 0; i < g.count; ++i)
            if (sorted[i].dep && !kDepShape[sorted[i].shape]) return false;
    } else {
        int pi = -1;
        for (int i = 0; i < g.count; ++i) {
            if (g.p[i].y != d.qkv) continue;
            if (pi >= 0 || g.p[i].y_dtype != MVLM_F32 || g.p[i].N != 3 * d.heads * d.head_dim) return false;
            pi = i;
        }
        if (pi < 0 || !kDepShape[g.p[pi].shape]) return false;
        sorted[n] = g.p[pi];
        sorted[n++].prod = 1;
        for (int i = 0; i < g.count; ++i)
            if (i != pi) sorted[n++] = g.p[i];
    }
    for (int i = 0; i < g.count; ++i) g.p[i] = sorted[i];
    lds = std::max(lds, (size_t)NWAVE * (d.head_dim + 2) * 4);
    return lds <= STREAM_LDS_MAX;
}

template <class F>
static hipError_t attn_capacity(StreamGroup& g, size_t lds, int num_cus) {
    int per_cu = 0;
    if (const hipError_t e = allow_dynamic_lds<gemv_stream_kernel<F, float, 1, true>>((int)STREAM_LDS_MAX);
        e != hipSuccess)
        return e;
    if (const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, gemv_stream_kernel<F, float, 1, true>, 64 * NWAVE, lds);
        e != hipSuccess)
        return e;
    partition(g);
    const int waiting = g.at.mode == 0 ? g.at.consumers : g.at.blocks;
    const bool fits = g.at.mode == 0 ? g.at.consumers <= ATTN_MAX_CONSUMERS
                                     : g.at.prod_blocks <= ATTN_MAX_PRODUCERS && g.at.prod_blocks > 0;
    return waiting < per_cu * num_cus && fits ? hipSuccess : hipErrorInvalidConfiguration;
}

static hipError_t build_group(StreamGroup& g, size_t& lds, int count, const void* const* xs, int x_dtype,
                              const mvlm_weight* const* ws, void* const* ys, const int* y_dtypes, int num_cus,
                              const Epilogue* eps, int M);

hipError_t stream_attn_check(int count, const void* const* xs, int x_dtype, const mvlm_weight* const* ws,
                             void* const* ys, const int* y_dtypes, const StreamAttnDesc& at, int num_cus) {
    StreamGroup g{};
    size_t lds = 0;
    if (const hipError_t e = build_group(g, lds, count, xs, x_dtype, ws, ys, y_dtypes, num_cus, nullptr, 1);
        e != hipSuccess)
        return e;
    if (!attach_attention(g, at, x_dtype, 1, num_cus, lds)) return hipErrorInvalidValue;
    switch (ws[0]->dtype) {
        case MVLM_Q8_0: return attn_capacity<Q8Fmt>(g, lds, num_cus);
        case MVLM_Q4_0: return attn_capacity<Q4Fmt>(g, lds, num_cus);
        case MVLM_F32: return attn_capacity<DenseFmt<float>>(g, lds, num_cus);
        case MVLM_F16: return attn_capacity<DenseFmt<__half>>(g, lds, num_cus);
        case MVLM_BF16: return attn_capacity<DenseFmt<__hip_bfloat16>>(g, lds, num_cus);
        default: return hipErrorInvalidValue;
    }
}

// A decode attention as launches of its own: the split kernel, then (more
// than one split) the merge kernel.
hipError_t launch_attn_decode(hipStream_t s, const StreamAttnDesc& d, int num_cus) {
    StreamAttn a;
    if (!attn_fill(a, d, num_cus > 0 ? num_cus : 256)) return hipErrorInvalidValue;
    a.merge = 0;
    const bool two = a.splits > 1;
    if (!two) {
        if (a.D == 64) launch_kernel(attn_split_kernel<64>, dim3(a.blocks), dim3(64 * NWAVE), 0, s, a);
        else launch_kernel(attn_split_kernel<128>, dim3(a.blocks), dim3(64 * NWAVE), 0, s, a);
    } else {
        if (a.D == 64)
            launch_kernel_part(LaunchPart::First, attn_split_kernel<64>, dim3(a.blocks), dim3(64 * NWAVE), 0, s, a);
        else
            launch_kernel_part(LaunchPart::First, attn_split_kernel<128>, dim3(a.blocks), dim3(64 * NWAVE), 0, s, a);
        if (a.D == 64) launch_kernel_part(LaunchPart::Last, attn_merge_kernel<64>, dim3(a.heads), dim3(64), 0, s, a);
        else launch_kernel_part(LaunchPart::Last, attn_merge_kernel<128>, dim3(a.heads), dim3(64), 0, s, a);
    }
    return hipGetLastError();
}

// The launch's problems (validated by the caller) and its LDS bytes.
static hipError_t build_group(StreamGroup& g, size_t& lds, int count, const void* const* xs, int x_dtype,
                              const mvlm_weight* const* ws, void* const* ys, const int* y_dtypes, int num_cus,
                              const Epilogue* eps, int M) {
    if (count < 1 || count > MAX_GROUP || M < 1 || M > 4) return hipErrorInvalidValue;
    g.count = count;
    const int dtype = ws[0]->dtype;
    if (M > 1 && (!is_quant(dtype) || x_dtype != MVLM_F32)) return hipErrorInvalidValue;
    lds = 0;
    for (int i = 0; i < count; ++i) {
        const mvlm_weight* w = ws[i];
        StreamProblem& p = g.p[i];
        p.x = xs[i];
        p.codes = (const uint8_t*)w->data;
        p.scales = (const uint16_t*)w->scales;
        p.y = ys[i];
        p.ld_bytes = weight_row_bytes(w);
        p.N = w->N;
        p.K = w->K;
        p.y_dtype = y_dtypes[i];
        p.M = M;
        p.shape = stream_shape(w, M, num_cus > 0 ? num_cus : 256);
        if (eps && eps[i].any()) {
            p.ep = eps[i];
            p.ep_on = 1;
        }
        if (p.shape < 0 || w->dtype != dtype || (M > 1 && y_dtypes[i] != MVLM_F32)) return hipErrorInvalidValue;
        const size_t b = stream_lds_bytes(w, x_dtype, p.shape, batch_mx(M));
        lds = b > lds ? b : lds;
    }
    return lds > STREAM_LDS_MAX ? hipErrorInvalidValue : hipSuccess;
}

// All problems share the weight dtype and x dtype (checked by the caller).
// M > 1 (2..4 rows of fp32 x per problem, quantized weights) uses the
// batched-x kernel.  `at` (M = 1, fp32 x): the launch also computes that
// decode attention, whose output o is the x of some of the problems
// (stream_attn_check has accepted the combination).
hipError_t launch_gemv_stream_group(hipStream_t s, int count, const void* const* xs, int x_dtype,
                                    const mvlm_weight* const* ws, void* const* ys, const int* y_dtypes, int num_cus,
                                    const Epilogue* eps, int M, const StreamAttnDesc* at) {
    StreamGroup g{};
    size_t lds = 0;
    if (const hipError_t e = build_group(g, lds, count, xs, x_dtype, ws, ys, y_dtypes, num_cus, eps, M);
        e != hipSuccess)
        return e;
    const int dtype = ws[0]->dtype;
    if (at) {
        if (!attach_attention(g, *at, x_dtype, M, num_cus > 0 ? num_cus : 256, lds)) return hipErrorInvalidValue;
        switch (dtype) {
            case MVLM_Q8_0: return launch_group<Q8Fmt, float, 1, true>(s, g, lds);
            case MVLM_Q4_0: return launch_group<Q4Fmt, float, 1, true>(s, g, lds);
            case MVLM_F32: return launch_group<DenseFmt<float>, float, 1, true>(s, g, lds);
            case MVLM_F16: return launch_group<DenseFmt<__half>, float, 1, true>(s, g, lds);
            case MVLM_BF16: return launch_group<DenseFmt<__hip_bfloat16>, float, 1, true>(s, g, lds);
            default: return hipErrorInvalidValue;
        }
    }
    if (M == 2) return dtype == MVLM_Q8_0 ? launch_group<Q8Fmt, float, 2>(s, g, lds) : launch_group<Q4Fmt, float, 2>(s, g, lds);
    if (M > 2) return dtype == MVLM_Q8_0 ? launch_group<Q8Fmt, float, 4>(s, g, lds) : launch_group<Q4Fmt, float, 4>(s, g, lds);
    switch (dtype) {
        case MVLM_Q8_0: return launch_group<Q8Fmt, float>(s, g, lds);
        case MVLM_Q4_0: return launch_group<Q4Fmt, float>(s, g, lds);
        case MVLM_F32: return launch_group_x<DenseFmt<float>>(s, x_dtype, g, lds);
        case MVLM_F16: return launch_group_x<DenseFmt<__half>>(s, x_dtype, g, lds);
        case MVLM_BF16: return launch_group_x<DenseFmt<__hip_bfloat16>>(s, x_dtype, g, lds);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_stream(hipStream_t s, const void* x, int x_dtype, const mvlm_weight* W, void* y,
                              int y_dtype, int num_cus, const Epilogue* ep) {
    return launch_gemv_stream_group(s, 1, &x, x_dtype, &W, &y, &y_dtype, num_cus, ep);
}

// Quantized weight, fp32 x [M][K] and y [M][N], 2 <= M <= 4.
hipError_t launch_gemv_stream_batch(hipStream_t s, const float* x, const mvlm_weight* W, float* y, int M,
                                    int num_cus, const Epilogue* ep) {
    if (M < 2 || M > 4 || !stream_supported(W, M)) return hipErrorInvalidValue;
    StreamGroup g{};
    g.count = 1;
    StreamProblem& p = g.p[0];
    p.x = x;
    p.codes = (const uint8_t*)W->data;
    p.scales = (const uint16_t*)W->scales;
    p.y = y;
    p.ld_bytes = weight_row_bytes(W);
    p.N = W->N;
    p.K = W->K;
    p.y_dtype = MVLM_F32;
    p.M = M;
    p.shape = stream_shape(W, M, num_cus > 0 ? num_cus : 256);
    if (ep && ep->any()) {
        p.ep = *ep;
        p.ep_on = 1;
    }
    const size_t lds = stream_lds_bytes(W, MVLM_F32, p.shape, batch_mx(M));
    if (M == 2) {
        if (W->dtype == MVLM_Q8_0) return launch_group<Q8Fmt, float, 2>(s, g, lds);
        if (W->dtype == MVLM_Q4_0) return launch_group<Q4Fmt, float, 2>(s, g, lds);
    } else {
        if (W->dtype == MVLM_Q8_0) return launch_group<Q8Fmt, float, 4>(s, g, lds);
        if (W->dtype == MVLM_Q4_0) return launch_group<Q4Fmt, float, 4>(s, g, lds);
    }
    return hipErrorInvalidValue;
}

}  // namespace mvlm
