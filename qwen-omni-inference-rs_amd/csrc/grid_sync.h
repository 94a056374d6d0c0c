// grid_sync.h -- workgroup-to-workgroup hand-off for persistent kernels on
// gfx950 (8 XCDs, one L2 each, not coherent with each other for ordinary
// loads and stores of device memory).
//
// Two ways to make data written by one workgroup visible to another:
//   FENCED:  ordinary stores and loads; the arriving side runs an agent-scope
//            release (buffer_wbl2: the XCD's L2 writes its dirty lines back),
//            the waiting side an agent-scope acquire (buffer_inv: its L2 and
//            L1 drop their lines).
//   DIRECT:  the exchanged data itself is stored and loaded with agent-scope
//            atomic operations (global_store / global_load with sc1: written
//            through to, and read from, the device-coherent level), so no
//            cache-wide writeback or invalidate is needed; the arrive only
//            waits for the stores to complete (s_waitcnt) before counting.
// Counters are device-scope atomics in memory that only grows: the k-th
// synchronisation of a launch waits for the counter to reach k * parties,
// so nothing is reset between phases.
//
// Every wait is bounded: after SYNC_SPIN_LIMIT polls the waiter records an
// error bit and gives up, so a workgroup that never arrives (a launch whose
// workgroups are not all resident) ends the kernel instead of hanging it.
// Callers launch cooperatively (hipLaunchCooperativeKernel), which refuses a
// grid that cannot be co-resident.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lq8 {

constexpr unsigned SYNC_SPIN_LIMIT = 1u << 20;  // polls (each a memory round trip, then s_sleep 1) before giving up: ~1 s
constexpr int SYNC_XCDS = 8;
constexpr int SYNC_LINE = 64;  // u32 per 256-byte line: every counter on its own line

// Device memory of one synchronisation domain (zeroed once at allocation).
struct SyncState {
    unsigned count[SYNC_LINE];              // the grid counter (or the XCD leaders' counter)
    unsigned xcd[SYNC_XCDS][SYNC_LINE];     // per-XCD arrival counters
    unsigned flag[SYNC_XCDS][SYNC_LINE];    // per-XCD release flags (generation reached)
    unsigned err[SYNC_LINE];                // error bits: 1 = a wait gave up
};

__device__ __forceinline__ unsigned sync_load(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_store(unsigned* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned sync_add(unsigned* p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Coherent element access for DIRECT exchange.
__device__ __forceinline__ float xload(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xstore(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll until *p >= target (unsigned wrap-safe compare), bounded.
__device__ __forceinline__ bool sync_wait(const unsigned* p, unsigned target, unsigned* err) {
    unsigned spins = 0;
    while ((int)(sync_load(p) - target) < 0) {
        if (++spins > SYNC_SPIN_LIMIT) {
            __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

enum SyncKind : int {
    SYNC_FLAT_FENCED = 0,   // one counter, release/acquire fences
    SYNC_FLAT_DIRECT = 1,   // one counter, no cache-wide fences (DIRECT data)
    SYNC_XCD_DIRECT = 2,    // per-XCD counters, XCD leaders count globally, all poll the global counter
    SYNC_XCD_FLAGS = 3,     // per-XCD counters, the last leader raises 8 per-XCD flags, each XCD polls its own
};

// Grid-wide barrier number `gen` (1, 2, ...) of `nwg` workgroups.  Every
// thread of every workgroup calls it.  Before it, each thread's own global
// stores must have been issued; the function waits for them (s_waitcnt)
// before the workgroup arrives.  Returns false (in every thread) when a wait
// gave up.  Workgroup w is assumed to run on XCD w % 8 (the dispatcher's
// round-robin); the XCD variants are correct for any placement, only their
// contention depends on it.
template <int KIND>
__device__ __forceinline__ bool grid_sync(SyncState* s, unsigned gen, int nwg) {
    __shared__ int ok_s;
    if (KIND == SYNC_FLAT_FENCED) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        bool ok = true;
        if (KIND == SYNC_FLAT_FENCED) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        if (KIND == SYNC_FLAT_FENCED || KIND == SYNC_FLAT_DIRECT) {
            sync_add(s->count, 1u);
            ok = sync_wait(s->count, gen * (unsigned)nwg, s->err);
        } else {
            const int x = blockIdx.x & (SYNC_XCDS - 1);
            const unsigned nx = (unsigned)((nwg - x + SYNC_XCDS - 1) / SYNC_XCDS);
            const unsigned nlead = (unsigned)(nwg < SYNC_XCDS ? nwg : SYNC_XCDS);
            const unsigned old = sync_add(s->xcd[x], 1u);
            if (KIND == SYNC_XCD_DIRECT) {
                if (old + 1 == gen * nx) sync_add(s->count, 1u);
                ok = sync_wait(s->count, gen * nlead, s->err);
            } else {
                if (old + 1 == gen * nx) {
                    const unsigned o2 = sync_add(s->count, 1u);
                    if (o2 + 1 == gen * nlead)
                        for (int i = 0; i < (int)nlead; i++) sync_store(s->flag[i], gen);
                }
                ok = sync_wait(s->flag[x], gen, s->err);
            }
        }
        if (KIND == SYNC_FLAT_FENCED) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        ok_s = ok ? 1 : 0;
    }
    __syncthreads();
    return ok_s != 0;
}

}  // namespace lq8
