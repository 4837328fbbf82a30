// Persistent decode step: a chain of dependent grouped GEMV stages (M = 1,
// Q8_0 / Q4_0 weights, fp32 x and y) in one launch.
//
// A Phi-1.5 decode step is 49 dependent launches of the streaming GEMV
// (gemv_stream.hip): per layer {QKV, fc1} and {dense, fc2}, then the LM head
// (the projections of src/models/moondream2.cpp:369-541).  Each launch pays a
// fixed cost of ~3.5 us that moves no data: the dispatch ramp, the first
// requests' latency and the tail of the slowest CU, with HBM idle in between.
// Here one workgroup per CU lives for the whole step and the stage boundary
// becomes a grid-wide wait on per-block flags, while the weights of the next
// stages are already in flight: weights do not depend on the previous stage,
// only x does.
//
// Workgroup = CH_CWAVES compute waves + 1 leader wave.
//  * Compute waves own "rounds": up to 8 KiB of one problem's rows (R rows of
//    C 1 KiB chunks, R * C = 8) whose codes go straight into registers and
//    whose block scales go into the wave's LDS slot with direct loads.  Each
//    wave keeps two rounds in flight (double-buffered registers), across stage
//    boundaries, and writes each row's sum into the block's LDS y area.  Its
//    vector-memory counter only ever holds weight loads, so waiting for a round
//    never waits for anything else.
//  * The leader wave waits for every block's flag of the previous stage,
//    stages the stage's x into LDS, and after the compute waves are done stores
//    the block's y rows (epilogue applied), waits for those stores and raises
//    the block's flag.
// Cross-XCD visibility without cache flushes: y, the epilogue operands, x and
// the flags go through agent-scope (sc1) stores and loads, which bypass the
// per-XCD L2's non-coherent copies; the weights are plain loads.  Every wait is
// bounded (ChainArgs::timeout_ticks of the 100 MHz clock): on expiry the block records an error
// and leaves, so a broken chain ends instead of hanging.
//
// The compute waves issue every memory operation through inline asm the
// compiler does not track (device_math.h) and order them with explicit
// waits: the compiler's own waits would put vmcnt(0) in front of each LDS
// read (it cannot tell the scale slots from the x area) and drain the
// prefetched round.
#include "gemv_common.h"

#include <algorithm>
#include <new>
#include <vector>

namespace mvlm {

constexpr int CH_CWAVES = 7;                        // compute waves per workgroup
constexpr int CH_WAVES = CH_CWAVES + 1;             // + the leader (the last wave)
constexpr int CH_LOADS = 8;                         // 16-byte code loads per lane per round (8 KiB per wave)
constexpr int CH_SLOADS = 2;                        // 1 KiB direct scale loads per round
constexpr int CH_SLOT = CH_SLOADS * 1024;           // one scale slot (<= 1 KiB of scales + 16-byte alignment)
constexpr int CH_XMAX = 32 * 1024;                  // x bytes per stage (K <= 8192 fp32)
constexpr int CH_SXMAX = 1024;                      // Q4_0 block sums of x (K / 32 floats)
constexpr int CH_YMAX_ROWS = 512;                   // rows per block per stage
constexpr int CH_SEGS_BYTES = 128 * 48;             // the block's segment of each stage (CH_MAX_STAGES)
constexpr int CH_LDS = CH_XMAX + CH_SXMAX + CH_CWAVES * 2 * CH_SLOT + CH_YMAX_ROWS * 4 + CH_SEGS_BYTES;
// requesting more than half of the 160 KiB LDS keeps the workgroups one per CU
constexpr int CH_LDS_REQUEST = CH_LDS > 82 * 1024 ? CH_LDS : 82 * 1024;

struct ChainProblem {
    const float* x;            // [K]
    const uint8_t* codes;      // [N][ld_bytes]
    const uint16_t* scales;    // [N][K/32]
    float* y;                  // [N]
    int64_t ld_bytes;          // code bytes per row
    int N, K;
    int lg_chunks;             // log2 of the 1 KiB chunks per row (row bytes <= 2^lg_chunks KiB)
    int ep_on;
    Epilogue ep;               // fp32 operands
};

// A block's rows [row0, row1) of problem prob in one stage (prob < 0: none),
// with the fields the compute waves need copied out of the problem.
struct ChainSeg {
    const uint8_t* codes;
    const uint8_t* scales;
    int64_t ld;
    int prob, row0, row1, N, K, lg;
};
static_assert(sizeof(ChainSeg) == 48, "ChainSeg is copied to LDS as 12 dwords");
constexpr int CH_MAX_STAGES = 128;

struct ChainState {
    uint64_t epoch;            // launches completed
    uint32_t done;             // workgroups finished in this launch
    uint32_t error;            // nonzero once a wait gave up
    uint64_t pad[6];
};

struct ChainArgs {
    ChainState* state;
    uint64_t* flags;           // [nb]: epoch * 1024 + (last finished stage + 1)
    const ChainProblem* probs;
    const ChainSeg* segs;      // [stages][nb]
    int nb, stages;
    uint64_t timeout_ticks;    // s_memrealtime ticks (100 MHz) a wait may take before it gives up
};

// ---- agent-coherent memory access ----------------------------------------------

__device__ __forceinline__ uint64_t ld_agent(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// out = act(v + bias[n]) * mul[n] + res[n] with agent-coherent operand loads
// (an earlier stage of the chain may have written them)
__device__ __forceinline__ float chain_epilogue(const Epilogue& e, float v, int n) {
    if (e.bias) v += ld_agent((const float*)e.bias + n);
    if (e.act == 1) v = gelu_tanh(v);
    else if (e.act == 2) v = silu(v);
    if (e.mul) v *= ld_agent((const float*)e.mul + n);
    if (e.res) v += ld_agent((const float*)e.res + n);
    return v;
}

// x [K] fp32 into LDS with agent-coherent direct 16-byte loads (one wave), its
// 16-byte slots permuted by x_slot<SL> as the streaming kernel stores them.
template <int SL>
__device__ __forceinline__ void chain_stage_x(uint8_t* dst, const uint8_t* src, int nbytes, int lane) {
    for (int piece = 0; piece * 1024 < nbytes; ++piece) {
        const int phys = piece * 1024 + lane * 16;
        const int logical = x_slot<SL>(phys >> 4) * 16;
        const uint8_t* from = src + min(logical, nbytes - 16);
        __builtin_amdgcn_global_load_lds(from, (lds_void*)(dst + piece * 1024), 16, 0, 16 /* sc1 */);
    }
}

// Workgroup barrier ordering LDS only: the fences are limited to the local
// address space, so no wave waits for its outstanding global loads (which a
// full __syncthreads() would drain).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// untracked non-temporal 16-byte load (wait with asm_wait_vmcnt, then asm_pin)
__device__ __forceinline__ u32x4 asm_global_load_b128_nt(const void* p) {
    u32x4 v;
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(v) : "v"(p));
    return v;
}

template <class F>
struct ChainFmt {
    static constexpr bool Q4 = std::is_same_v<F, Q4Fmt>;
    static constexpr int WPL = F::WPL;                 // weights per lane per chunk
    static constexpr int SL = WPL * 4 / 16;            // 16-byte x slots per lane per chunk
};

// One round of a compute wave: nrows (<= CH_LOADS >> lg) consecutive rows of
// one problem, 2^lg chunks each.  Every field is wave-uniform.
struct RoundDesc {
    int stage;                 // -1: nothing left
    int nrows, lg, K;
    int ylo;                   // first row's index in the block's y area
    int soff;                  // first row's scale byte in the slot (below 16: alignment)
    int64_t ld;                // code bytes per row
    const uint8_t* codes;      // first row's codes
    const uint8_t* scales;     // 16-byte aligned start of the rows' scales
    const uint8_t* scale_last; // last 16-byte piece of the problem's scale array
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ const uint8_t* uni(const uint8_t* p) {
    return reinterpret_cast<const uint8_t*>(uni((int64_t)reinterpret_cast<uintptr_t>(p)));
}
__device__ __forceinline__ RoundDesc uniform(RoundDesc d) {
    d.stage = uni(d.stage); d.nrows = uni(d.nrows); d.lg = uni(d.lg); d.K = uni(d.K);
    d.ylo = uni(d.ylo); d.soff = uni(d.soff); d.ld = uni(d.ld);
    d.codes = uni(d.codes); d.scales = uni(d.scales); d.scale_last = uni(d.scale_last);
    return d;
}

// untracked LDS dword read (wait with asm_wait_lgkmcnt, then asm_pin)
__device__ __forceinline__ uint32_t asm_lds_read_b32(uint32_t addr) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

template <class F>
__global__ __launch_bounds__(64 * CH_WAVES, 1) void gemv_chain_kernel(const ChainArgs a) {
    using CF = ChainFmt<F>;
    constexpr int SL = CF::SL;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    uint8_t* xl = lds;
    float* sxl = reinterpret_cast<float*>(lds + CH_XMAX);
    uint8_t* slots = lds + CH_XMAX + CH_SXMAX;
    float* yl = reinterpret_cast<float*>(slots + CH_CWAVES * 2 * CH_SLOT);
    ChainSeg* segl = reinterpret_cast<ChainSeg*>(reinterpret_cast<uint8_t*>(yl) + CH_YMAX_ROWS * 4);
    __shared__ uint64_t epoch_s;
    __shared__ int abort_s;

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int b = blockIdx.x, nb = a.nb;
    if (threadIdx.x == 0) {
        epoch_s = ld_agent(&a.state->epoch);
        abort_s = 0;
    }
    // this block's segment of every stage into LDS: the compute waves read it
    // there (a table read through vector memory would wait on vmcnt, which
    // holds their prefetched rounds)
    for (int i = threadIdx.x; i < a.stages * 12; i += 64 * CH_WAVES)
        reinterpret_cast<uint32_t*>(segl)[i] = reinterpret_cast<const uint32_t*>(a.segs + (i / 12) * nb + b)[i % 12];
    __syncthreads();
    const uint64_t E = epoch_s;

    if (wave == CH_CWAVES) {
        // ------------------------------------------------------------ leader
        for (int s = 0; s < a.stages; ++s) {
            const ChainSeg sg = segl[s];
            if (s > 0) {   // every block's flag must show stage s-1 finished
                const uint64_t want = E * 1024 + (uint64_t)s;
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                bool ok = false;
                while (true) {
                    bool mine = true;
                    for (int i = lane; i < nb; i += 64) mine &= ld_agent(&a.flags[i]) >= want;
                    ok = __builtin_amdgcn_ballot_w64(!mine) == 0;
                    if (ok || __builtin_amdgcn_s_memrealtime() - t0 > a.timeout_ticks) break;
                    __builtin_amdgcn_s_sleep(1);
                }
                if (!ok) {
                    if (lane == 0) {
                        __hip_atomic_store(&a.state->error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        abort_s = 1;
                    }
                    lds_barrier();   // releases the compute waves, which see abort_s
                    return;
                }
            }
            if (sg.prob >= 0) {
                const ChainProblem& P = a.probs[sg.prob];
                chain_stage_x<SL>(xl, reinterpret_cast<const uint8_t*>(P.x), P.K * 4, lane);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                if constexpr (CF::Q4) {   // block sums of x (the -8 offset's term), once per block and stage
                    for (int blk = lane; blk < (P.K >> 5); blk += 64) {
                        XRaw<float, 32> xr;
#pragma unroll
                        for (int v = 0; v < SL; ++v) {
                            const u32x4 u = reinterpret_cast<const u32x4*>(xl)[x_slot<SL>(SL * blk + v)];
                            xr.d[4 * v + 0] = u[0]; xr.d[4 * v + 1] = u[1];
                            xr.d[4 * v + 2] = u[2]; xr.d[4 * v + 3] = u[3];
                        }
                        sxl[blk] = x_block_sum(xr);
                    }
                }
            }
            lds_barrier();   // A(s): x staged
            lds_barrier();   // B(s): rows computed
            if (sg.prob >= 0) {
                const ChainProblem& P = a.probs[sg.prob];
                for (int i = lane; i < sg.row1 - sg.row0; i += 64) {
                    const int n = sg.row0 + i;
                    float v = yl[i];
                    if (P.ep_on) v = chain_epilogue(P.ep, v, n);
                    st_agent(P.y + n, v);
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            if (lane == 0) st_agent(&a.flags[b], E * 1024 + (uint64_t)(s + 1));
        }
        if (lane == 0) {   // the last workgroup to finish closes the launch
            const uint32_t old = __hip_atomic_fetch_add(&a.state->done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old == (uint32_t)nb - 1) {
                __hip_atomic_store(&a.state->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&a.state->epoch, E + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        return;
    }

    // --------------------------------------------------------------- compute
    // This wave's rounds: in stage s, the block's rows split into rounds of R
    // rows, round j going to wave j % CH_CWAVES; stages in order.  Every round
    // descriptor field is wave-uniform (scalar registers), so no table read in
    // the loop goes through the vector memory counter.
    int cur_s = 0, cur_j = wave;
    auto next_round = [&]() -> RoundDesc {
        while (true) {
            cur_s = uni(cur_s);
            cur_j = uni(cur_j);
            if (cur_s >= a.stages) break;
            const ChainSeg& sg = segl[cur_s];
            const int prob = uni(sg.prob);
            if (prob >= 0) {
                const int lg = uni(sg.lg), row0 = uni(sg.row0), row1 = uni(sg.row1);
                const int R = CH_LOADS >> lg;
                const int rs = row0 + cur_j * R;
                if (rs < row1) {
                    RoundDesc d;
                    d.stage = cur_s;
                    d.nrows = min(R, row1 - rs);
                    d.lg = lg;
                    d.K = sg.K;
                    d.ylo = rs - row0;
                    d.ld = sg.ld;
                    d.codes = sg.codes + (int64_t)rs * sg.ld;
                    const int64_t sb = (int64_t)(sg.K >> 5) * 2;
                    const int64_t s0 = ((int64_t)rs * sb) & ~(int64_t)15;
                    const int64_t s_last = ((int64_t)sg.N * sb - 16) & ~(int64_t)15;
                    d.soff = (int)((int64_t)rs * sb - s0);
                    d.scales = sg.scales + s0;
                    d.scale_last = sg.scales + (s_last > 0 ? s_last : 0);
                    cur_j += CH_CWAVES;
                    return uniform(d);
                }
            }
            ++cur_s;
            cur_j = wave;
        }
        RoundDesc d{};
        d.stage = -1;
        d.codes = d.scales = d.scale_last = reinterpret_cast<const uint8_t*>(a.state);   // any readable bytes
        return uniform(d);
    };

    // Loads of one round: CH_LOADS code vectors (rows past the round's last
    // row repeat it, lanes past a row's end load its first vector: always in
    // bounds) and the rows' block scales (direct loads into the slot, clamped
    // to the array's last 16 bytes).  An empty round loads harmless bytes, so
    // every round adds the same count to vmcnt.
    auto issue = [&](const RoundDesc& d, u32x4 (&q)[CH_LOADS], int slot_idx) {
        int lane = threadIdx.x & 63;     // (not hoisted: see compute)
        asm volatile("" : "+v"(lane));
        const uint32_t slot = __builtin_amdgcn_readfirstlane(lds_offset(slots + (wave * 2 + slot_idx) * CH_SLOT));
        // slot t holds chunk t & (C - 1) of row t >> lg
        const int lgmask = (1 << d.lg) - 1;
#pragma unroll
        for (int t = 0; t < CH_LOADS; ++t) {
            const int row = min(t >> d.lg, d.nrows - 1);
            const int64_t off = (int64_t)((t & lgmask) * 1024 + lane * 16);
            q[t] = asm_global_load_b128_nt(d.codes + (int64_t)row * d.ld + (off < d.ld ? off : 0));
        }
#pragma unroll
        for (int i = 0; i < CH_SLOADS; ++i) {
            const uint8_t* src = d.scales + i * 1024 + lane * 16;
            asm_global_load_lds_b128(src < d.scale_last ? src : d.scale_last, slot + i * 1024);
        }
    };

    // Rows of one round: x chunk by chunk from LDS (shared by the rows), codes
    // from registers, scales from the slot; row sums into the LDS y area.
    const uint32_t xl_off = lds_offset(xl), sxl_off = lds_offset(sxl);
    auto compute = [&](const RoundDesc& d, const u32x4 (&q)[CH_LOADS], int slot_idx, auto LG) {
        constexpr int LGC = decltype(LG)::value, C = 1 << LGC, R = CH_LOADS >> LGC;
        // lane-derived addresses are recomputed per round: hoisted out of the
        // round loop they would hold dozens of registers for its whole length
        int lane = threadIdx.x & 63;
        asm volatile("" : "+v"(lane));
        const uint32_t slot = lds_offset(slots + (wave * 2 + slot_idx) * CH_SLOT);
        const int sb = (d.K >> 5) * 2;
        const int xt = ((lane * SL) >> 4) & (SL - 1);
        float acc[R];
#pragma unroll
        for (int i = 0; i < R; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const int k = (64 * c + lane) * CF::WPL;
            const bool valid = k < d.K;
            const uint32_t xb = xl_off + (valid ? (64 * c + lane) * SL * 16 : 0);
            u32x4 xu[SL];
#pragma unroll
            for (int v = 0; v < SL; ++v) xu[v] = asm_lds_read_b128(xb + ((v ^ xt) << 4));
            uint32_t dh[R];
            const uint32_t sbase = slot + d.soff + (valid ? (k >> 5) * 2 : 0);
#pragma unroll
            for (int i = 0; i < R; ++i) dh[i] = asm_lds_read_u16(sbase + i * sb);
            uint32_t sxu = 0;
            if constexpr (CF::Q4) sxu = asm_lds_read_b32(sxl_off + (valid ? (k >> 5) * 4 : 0));
            asm_wait_lgkmcnt<0>();
#pragma unroll
            for (int v = 0; v < SL; ++v) asm_pin(xu[v]);
#pragma unroll
            for (int i = 0; i < R; ++i) asm_pin(dh[i]);
            asm_pin(sxu);
            XRaw<float, CF::WPL> xr;
#pragma unroll
            for (int v = 0; v < SL; ++v) {
                xr.d[4 * v + 0] = xu[v][0]; xr.d[4 * v + 1] = xu[v][1];
                xr.d[4 * v + 2] = xu[v][2]; xr.d[4 * v + 3] = xu[v][3];
            }
#pragma unroll
            for (int i = 0; i < R; ++i) {
                float v;
                if constexpr (CF::Q4) v = chunk_dot_q4(q[i * C + c], (uint16_t)dh[i], xr, __uint_as_float(sxu), acc[i]);
                else v = chunk_dot(F{}, q[i * C + c], (uint16_t)dh[i], xr, acc[i]);
                acc[i] = valid ? v : acc[i];
            }
        }
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const float v = wave_sum(acc[i]);
            if (lane == 0 && i < d.nrows) yl[d.ylo + i] = v;
        }
    };
    auto compute_any = [&](const RoundDesc& d, const u32x4 (&q)[CH_LOADS], int slot_idx) {
        switch (d.lg) {
            case 0: compute(d, q, slot_idx, std::integral_constant<int, 0>{}); break;
            case 1: compute(d, q, slot_idx, std::integral_constant<int, 1>{}); break;
            case 2: compute(d, q, slot_idx, std::integral_constant<int, 2>{}); break;
            default: compute(d, q, slot_idx, std::integral_constant<int, 3>{}); break;
        }
    };

    // Two round buffers in fixed registers, consumed alternately (q0, q1, q0,
    // ...; the oldest outstanding round is always the one about to be
    // computed).  Before a round of stage s the wave passes the workgroup
    // barriers of every stage up to s: B (y rows written) of the previous one
    // and A (x staged) of the next, so all waves pass the same barriers in the
    // same order whatever their share of rounds.
    u32x4 q0[CH_LOADS], q1[CH_LOADS];
    RoundDesc r0 = next_round();
    issue(r0, q0, 0);
    RoundDesc r1 = next_round();
    issue(r1, q1, 1);
    constexpr int PER_ROUND = CH_LOADS + CH_SLOADS;
    int at = -1;                        // last stage whose barrier A this wave passed
    auto advance_to = [&](int s) -> bool {   // false: the leader gave up
        while (at < s) {
            if (at >= 0) lds_barrier();       // B(at)
            ++at;
            lds_barrier();                    // A(at)
            // (an untracked LDS read: a generic or volatile access would be a
            // flat load, whose wait also drains the prefetched rounds)
            const uint32_t ab = asm_lds_read_b32(lds_offset(&abort_s));
            asm_wait_lgkmcnt<0>();
            if (__builtin_amdgcn_readfirstlane(ab) != 0) return false;
        }
        return true;
    };
    bool ok = true;
    while (true) {
        if (r0.stage < 0) break;
        if (!advance_to(r0.stage)) { ok = false; break; }
        asm_wait_vmcnt<PER_ROUND>();      // q0's round (q1's round, issued later, stays in flight)
#pragma unroll
        for (int t = 0; t < CH_LOADS; ++t) asm_pin(q0[t]);
        compute_any(r0, q0, 0);
        asm_wait_lgkmcnt<0>();            // the slot's reads are done before its refill
        r0 = next_round();
        issue(r0, q0, 0);
        if (r1.stage < 0) break;
        if (!advance_to(r1.stage)) { ok = false; break; }
        asm_wait_vmcnt<PER_ROUND>();
#pragma unroll
        for (int t = 0; t < CH_LOADS; ++t) asm_pin(q1[t]);
        compute_any(r1, q1, 1);
        asm_wait_lgkmcnt<0>();
        r1 = next_round();
        issue(r1, q1, 1);
    }
    // The trailing rounds are in flight into registers the compiler considers
    // free from here on: let them land first.
    asm_wait_vmcnt<0>();
    if (ok && advance_to(a.stages - 1)) lds_barrier();   // the remaining barriers, B(last) included
}

// ---- host side -------------------------------------------------------------------

static int lg2_exact(int64_t v) {
    int l = 0;
    while ((int64_t)1 << l < v) ++l;
    return ((int64_t)1 << l) == v ? l : -1;
}

// Quantized weights whose rows are a power-of-two count of 1 KiB chunks (at
// most CH_LOADS) and whose fp32 x fits the staged area.
bool chain_supported(const mvlm_weight* w) {
    if (!is_quant(w->dtype) || w->K % 32 != 0) return false;
    const int64_t chunks = (w->ld + 1023) / 1024;
    if (lg2_exact(chunks) < 0 || chunks > CH_LOADS) return false;
    return (int64_t)w->K * 4 <= CH_XMAX;
}

struct ChainPlan {
    int dtype = 0;
    int nb = 0, stages = 0;
    void* mem = nullptr;       // state + flags + problems + segments
    ChainArgs args{};
};

int chain_build(const std::vector<std::vector<ChainEntry>>& stages, int num_cus, ChainPlan** out) {
    *out = nullptr;
    if (stages.empty()) return set_error(MVLM_ERR_INVALID_ARG, "chain: no stages");
    const int nb = num_cus > 0 ? num_cus : 256;
    const int dtype = stages[0][0].w->dtype;
    std::vector<ChainProblem> probs;
    ChainSeg none{};
    none.prob = -1;
    std::vector<ChainSeg> segs((size_t)stages.size() * nb, none);
    if (stages.size() > (size_t)CH_MAX_STAGES)
        return set_error(MVLM_ERR_UNSUPPORTED, "chain: %zu stages exceed %d", stages.size(), CH_MAX_STAGES);
    for (size_t s = 0; s < stages.size(); ++s) {
        const auto& st = stages[s];
        // blocks per problem in proportion to its bytes (at least one each)
        double total = 0.0;
        for (const ChainEntry& e : st) total += (double)e.w->N * (double)e.w->ld;
        std::vector<int> share(st.size());
        int given = 0;
        for (size_t i = 0; i < st.size(); ++i) {
            share[i] = std::max(1, (int)((double)nb * (double)st[i].w->N * (double)st[i].w->ld / total));
            share[i] = std::min(share[i], st[i].w->N);
            given += share[i];
        }
        while (given > nb) {   // trim the largest shares
            size_t big = 0;
            for (size_t i = 1; i < st.size(); ++i) if (share[i] > share[big]) big = i;
            if (share[big] <= 1) return set_error(MVLM_ERR_UNSUPPORTED, "chain: stage %zu has more problems than CUs", s);
            --share[big];
            --given;
        }
        while (given < nb) {   // add to the problem with the most rows per block
            size_t best = 0;
            double most = -1.0;
            for (size_t i = 0; i < st.size(); ++i) {
                const double per = (double)st[i].w->N * st[i].w->ld / share[i];
                if (share[i] < st[i].w->N && per > most) { most = per; best = i; }
            }
            if (most < 0) break;
            ++share[best];
            ++given;
        }
        int blk = 0;
        for (size_t i = 0; i < st.size(); ++i) {
            const ChainEntry& e = st[i];
            ChainProblem p{};
            p.x = (const float*)e.x;
            p.codes = (const uint8_t*)e.w->data;
            p.scales = (const uint16_t*)e.w->scales;
            p.y = (float*)e.y;
            p.ld_bytes = e.w->ld;
            p.N = e.w->N;
            p.K = e.w->K;
            p.lg_chunks = lg2_exact((e.w->ld + 1023) / 1024);
            if (e.ep.any()) {
                p.ep = e.ep;
                p.ep_on = 1;
            }
            const int pi = (int)probs.size();
            probs.push_back(p);
            for (int k = 0; k < share[i]; ++k, ++blk) {
                const int r0 = (int)((int64_t)e.w->N * k / share[i]);
                const int r1 = (int)((int64_t)e.w->N * (k + 1) / share[i]);
                if (r1 - r0 > CH_YMAX_ROWS)
                    return set_error(MVLM_ERR_UNSUPPORTED, "chain: %d rows per block exceed %d", r1 - r0, CH_YMAX_ROWS);
                ChainSeg g{};
                g.codes = p.codes;
                g.scales = reinterpret_cast<const uint8_t*>(p.scales);
                g.ld = p.ld_bytes;
                g.prob = pi;
                g.row0 = r0;
                g.row1 = r1;
                g.N = p.N;
                g.K = p.K;
                g.lg = p.lg_chunks;
                segs[s * nb + blk] = g;
            }
        }
    }
    const size_t off_flags = sizeof(ChainState);
    const size_t off_probs = (off_flags + (size_t)nb * 8 + 255) & ~(size_t)255;
    const size_t off_segs = (off_probs + probs.size() * sizeof(ChainProblem) + 255) & ~(size_t)255;
    const size_t bytes = off_segs + segs.size() * sizeof(ChainSeg);
    ChainPlan* cp = new (std::nothrow) ChainPlan();
    if (!cp) return set_error(MVLM_ERR_OUT_OF_MEMORY, "chain: host allocation failed");
    if (hipMalloc(&cp->mem, bytes) != hipSuccess) {
        (void)hipGetLastError();
        delete cp;
        return set_error(MVLM_ERR_OUT_OF_MEMORY, "chain: device allocation of %zu bytes failed", bytes);
    }
    char* base = (char*)cp->mem;
    int st = check_hip(hipMemset(base, 0, off_probs), "chain state");
    if (st == MVLM_OK) st = check_hip(hipMemcpy(base + off_probs, probs.data(), probs.size() * sizeof(ChainProblem),
                                                hipMemcpyHostToDevice), "chain problems");
    if (st == MVLM_OK) st = check_hip(hipMemcpy(base + off_segs, segs.data(), segs.size() * sizeof(ChainSeg),
                                                hipMemcpyHostToDevice), "chain segments");
    if (st != MVLM_OK) {
        (void)hipFree(cp->mem);
        delete cp;
        return st;
    }
    cp->dtype = dtype;
    cp->nb = nb;
    cp->stages = (int)stages.size();
    cp->args.state = (ChainState*)base;
    cp->args.flags = (uint64_t*)(base + off_flags);
    cp->args.probs = (const ChainProblem*)(base + off_probs);
    cp->args.segs = (const ChainSeg*)(base + off_segs);
    cp->args.nb = nb;
    cp->args.stages = (int)stages.size();
    cp->args.timeout_ticks = 2000000;   // 20 ms at 100 MHz: a stage takes well under 1 ms
    *out = cp;
    return MVLM_OK;
}

void chain_free(ChainPlan* cp) {
    if (!cp) return;
    if (cp->mem) (void)hipFree(cp->mem);
    delete cp;
}

hipError_t launch_chain(hipStream_t s, const ChainPlan* cp) {
    if (cp->dtype == MVLM_Q8_0) {
        if (const hipError_t e = allow_dynamic_lds<gemv_chain_kernel<Q8Fmt>>(CH_LDS_REQUEST); e != hipSuccess) return e;
        launch_kernel(gemv_chain_kernel<Q8Fmt>, dim3(cp->nb), dim3(64 * CH_WAVES), CH_LDS_REQUEST, s, cp->args);
    } else {
        if (const hipError_t e = allow_dynamic_lds<gemv_chain_kernel<Q4Fmt>>(CH_LDS_REQUEST); e != hipSuccess) return e;
        launch_kernel(gemv_chain_kernel<Q4Fmt>, dim3(cp->nb), dim3(64 * CH_WAVES), CH_LDS_REQUEST, s, cp->args);
    }
    return hipGetLastError();
}

int chain_error(const ChainPlan* cp, uint32_t* error) {
    HIP_TRY(hipMemcpy(error, &cp->args.state->error, 4, hipMemcpyDeviceToHost));
    return MVLM_OK;
}

}  // namespace mvlm
