// Grid-wide barrier latency probe (mvlm_probe_grid_barrier).
//
// A decode step is 49 dependent launches; a kernel boundary costs ~3.5 us of
// HBM time.  The alternative is one persistent launch whose workgroups
// synchronise through memory between stages.  This probe measures what such
// a software grid barrier costs on the device: one workgroup per CU runs
// `rounds` barriers back to back, each preceded by a 256-byte agent-coherent
// store and its wait (a stage's published outputs), optionally while the
// workgroup's other 8 waves stream HBM (the weights of the next stages).
// Arrival/wait protocols:
//   0  one counter per round, returning atomic add, then polls of the counter
//   1  one flag per workgroup on its own 128-byte line; every workgroup polls
//      all flags
//   2  returning atomic add; the last arriver raises a done flag replicated on
//      32 lines, each workgroup polls its replica
// Every wait is bounded (20 ms); a round that gives up ends the workgroup's
// rounds and is reported as MVLM_ERR_HIP.
#include "common.h"

#include <vector>

namespace mvlm {

typedef unsigned int p32x4 __attribute__((ext_vector_type(4)));

struct ProbeArgs {
    uint32_t* cnt;             // [rounds * 64]
    uint32_t* flags;           // [nb * 32]
    uint32_t* done;            // [rounds * 32 * 32]
    float* y;                  // [nb * 64]
    const p32x4* bg;           // background stream source
    uint64_t bg_n;             // its 16-byte elements
    uint32_t* err;
    uint64_t* ticks;           // [nb] s_memrealtime ticks of each workgroup's rounds
    int nb, rounds, variant, background;
};

constexpr uint64_t PROBE_TIMEOUT = 2000000;   // 20 ms at 100 MHz

__device__ __forceinline__ uint32_t probe_ld(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void probe_st(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(576, 1) void probe_barrier_kernel(ProbeArgs a) {
    __shared__ uint32_t stop;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, b = blockIdx.x;
    if (threadIdx.x == 0) stop = 0;
    __syncthreads();
    if (wave > 0) {   // background: 8 waves streaming HBM until wave 0 is done
        if (!a.background) return;
        p32x4 acc = {0, 0, 0, 0};
        uint64_t i = ((uint64_t)b * 8 + wave) * 64 * 16 + lane;
        for (int it = 0; it < 1000000; ++it) {
            if (__hip_atomic_load(&stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) break;
            p32x4 v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = __builtin_nontemporal_load(a.bg + (i + u * 64) % a.bg_n);
#pragma unroll
            for (int u = 0; u < 16; ++u) acc ^= v[u];
            i += (uint64_t)a.nb * 8 * 64 * 16;
        }
        if (acc[0] == 0x9E3779B9u && acc[1] == 0x7F4A7C15u) a.err[1] = 1;   // keeps the loads
        return;
    }
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    bool ok = true;
    for (int r = 0; r < a.rounds && ok; ++r) {
        probe_st(reinterpret_cast<uint32_t*>(a.y + b * 64 + lane), (uint32_t)r);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const uint64_t ts = __builtin_amdgcn_s_memrealtime();
        if (a.variant == 0) {
            uint32_t* c = a.cnt + r * 64;
            uint32_t now = 0;
            if (lane == 0) now = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
            now = __builtin_amdgcn_readfirstlane(now);
            while (now < (uint32_t)a.nb) {
                if (__builtin_amdgcn_s_memrealtime() - ts > PROBE_TIMEOUT) { ok = false; break; }
                __builtin_amdgcn_s_sleep(1);
                now = __builtin_amdgcn_readfirstlane(probe_ld(c));
            }
        } else if (a.variant == 1) {
            if (lane == 0) probe_st(a.flags + b * 32, (uint32_t)(r + 1));
            while (true) {
                bool mine = true;
                for (int i = lane; i < a.nb; i += 64) mine &= probe_ld(a.flags + i * 32) >= (uint32_t)(r + 1);
                if (__builtin_amdgcn_ballot_w64(!mine) == 0) break;
                if (__builtin_amdgcn_s_memrealtime() - ts > PROBE_TIMEOUT) { ok = false; break; }
                __builtin_amdgcn_s_sleep(1);
            }
        } else {
            uint32_t* c = a.cnt + r * 64;
            uint32_t now = 0;
            if (lane == 0) now = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
            now = __builtin_amdgcn_readfirstlane(now);
            uint32_t* d = a.done + (uint64_t)r * 32 * 32;
            if (now == (uint32_t)a.nb) {
                if (lane < 32) probe_st(d + lane * 32, 1u);
            } else {
                while (__builtin_amdgcn_readfirstlane(probe_ld(d + (b & 31) * 32)) == 0) {
                    if (__builtin_amdgcn_s_memrealtime() - ts > PROBE_TIMEOUT) { ok = false; break; }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
        }
    }
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    if (lane == 0) {
        a.ticks[b] = t1 - t0;
        if (!ok) probe_st(a.err, 1u);
        __hip_atomic_store(&stop, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

}  // namespace mvlm

using namespace mvlm;

extern "C" int mvlm_probe_grid_barrier(mvlm_device* dev, int variant, int rounds, int background,
                                       double* us_per_round) {
    REQUIRE(dev && us_per_round, "mvlm_probe_grid_barrier: null argument");
    REQUIRE(variant >= 0 && variant <= 2, "mvlm_probe_grid_barrier: variant %d not in 0..2", variant);
    REQUIRE(rounds >= 1 && rounds <= 1000, "mvlm_probe_grid_barrier: rounds %d not in 1..1000", rounds);
    HIP_TRY(hipSetDevice(dev->ordinal));
    const int nb = dev->prop.multiProcessorCount;
    const size_t bg_bytes = background ? ((size_t)512 << 20) : 4096;
    const size_t off_flags = (size_t)rounds * 64 * 4;
    const size_t off_done = off_flags + (size_t)nb * 32 * 4;
    const size_t off_y = off_done + (size_t)rounds * 32 * 32 * 4;
    const size_t off_err = off_y + (size_t)nb * 64 * 4;
    const size_t off_ticks = off_err + 256;
    const size_t off_bg = (off_ticks + (size_t)nb * 8 + 4095) & ~(size_t)4095;
    const size_t total = off_bg + bg_bytes;
    char* mem = nullptr;
    HIP_TRY(hipMalloc(&mem, total));
    int st = check_hip(hipMemset(mem, 0, total), "probe memset");
    ProbeArgs a{};
    a.cnt = (uint32_t*)mem;
    a.flags = (uint32_t*)(mem + off_flags);
    a.done = (uint32_t*)(mem + off_done);
    a.y = (float*)(mem + off_y);
    a.err = (uint32_t*)(mem + off_err);
    a.ticks = (uint64_t*)(mem + off_ticks);
    a.bg = (const p32x4*)(mem + off_bg);
    a.bg_n = bg_bytes / 16;
    a.nb = nb;
    a.rounds = rounds;
    a.variant = variant;
    a.background = background ? 1 : 0;
    if (st == MVLM_OK) {
        // 96 KiB of LDS keeps the workgroups one per CU
        st = check_hip(hipFuncSetAttribute((const void*)probe_barrier_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024), "probe attribute");
    }
    if (st == MVLM_OK) {
        hipLaunchKernelGGL(probe_barrier_kernel, dim3(nb), dim3(576), 96 * 1024, dev->stream, a);
        st = check_hip(hipGetLastError(), "probe launch");
    }
    if (st == MVLM_OK) st = check_hip(hipStreamSynchronize(dev->stream), "probe sync");
    std::vector<uint64_t> ticks((size_t)nb);
    uint32_t err = 0;
    if (st == MVLM_OK) st = check_hip(hipMemcpy(ticks.data(), a.ticks, (size_t)nb * 8, hipMemcpyDeviceToHost), "probe read");
    if (st == MVLM_OK) st = check_hip(hipMemcpy(&err, a.err, 4, hipMemcpyDeviceToHost), "probe read");
    (void)hipFree(mem);
    if (st != MVLM_OK) return st;
    if (err) return set_error(MVLM_ERR_HIP, "mvlm_probe_grid_barrier: a barrier wait gave up after 20 ms");
    uint64_t mx = 0;
    for (uint64_t t : ticks) mx = t > mx ? t : mx;
    *us_per_round = (double)mx / 100.0 / rounds;   // s_memrealtime: 100 MHz
    return MVLM_OK;
}
