// bench_sync.hip -- microbenchmark of the workgroup hand-off of grid_sync.h:
// the cost of one grid-wide synchronisation, with a data exchange checked
// every round, for each synchronisation kind and grid size.
#include <vector>

#include "grid_sync.h"
#include "lq8_internal.h"

namespace lq8 {

namespace {

// `rounds` rounds of: every workgroup writes 64 values of its own (round r,
// workgroup w: r * 4096 + w + lane / 64), a grid sync, every workgroup reads
// the 64 values of workgroup (w + r + 1) % nwg and counts mismatches, a grid
// sync (so the next round's writes do not overtake the reads).
template <int KIND>
__global__ __launch_bounds__(256) void k_sync_bench(SyncState* s, float* slots, int rounds, unsigned* mismatches) {
    const int nwg = gridDim.x, w = blockIdx.x, t = threadIdx.x;
    unsigned gen = 0, bad = 0;
    for (int r = 0; r < rounds; r++) {
        if (t < 64) {
            const float v = (float)(r * 4096 + w) + (float)t / 64.0f;
            if (KIND == SYNC_FLAT_FENCED) slots[w * 64 + t] = v;
            else xstore(slots + w * 64 + t, v);
        }
        if (!grid_sync<KIND>(s, ++gen, nwg)) return;
        if (t < 64) {
            const int src = (w + r + 1) % nwg;
            const float want = (float)(r * 4096 + src) + (float)t / 64.0f;
            const float got = KIND == SYNC_FLAT_FENCED ? slots[src * 64 + t] : xload(slots + src * 64 + t);
            bad += got != want;
        }
        if (!grid_sync<KIND>(s, ++gen, nwg)) return;
    }
    if (bad) atomicAdd(mismatches, bad);
}

template <int KIND>
hipError_t launch_bench(SyncState* s, float* slots, int rounds, unsigned* mism, int nwg, hipStream_t st) {
    void* args[] = {&s, &slots, &rounds, &mism};
    return hipLaunchCooperativeKernel((const void*)k_sync_bench<KIND>, dim3((unsigned)nwg), dim3(256), args, 0, st);
}

}  // namespace

}  // namespace lq8

using namespace lq8;

extern "C" lq8_status lq8_bench_grid_sync(lq8_ctx* ctx, int kind, int nwg, int rounds, float* us_per_sync,
                                          uint32_t* mismatches, uint32_t* gave_up) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid context handle");
    if (!us_per_sync || !mismatches || !gave_up) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (kind < SYNC_FLAT_FENCED || kind > SYNC_XCD_FLAGS) return fail(LQ8_ERR_INVALID_ARG, "unknown sync kind");
    if (nwg <= 0 || rounds <= 0 || rounds > 100000) return fail(LQ8_ERR_INVALID_ARG, "bad grid or round count");
    LQ8_HIP(hipSetDevice(ctx->device));
    int coop = 0;
    LQ8_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, ctx->device));
    if (!coop) return fail(LQ8_ERR_DEVICE, "device does not support cooperative launch");
    SyncState* s = nullptr;
    float* slots = nullptr;
    unsigned* mism = nullptr;
    hipError_t e = hipMalloc(&s, sizeof(SyncState));
    if (e == hipSuccess) e = hipMalloc(&slots, (size_t)nwg * 64 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&mism, sizeof(unsigned));
    if (e == hipSuccess) e = hipMemsetAsync(s, 0, sizeof(SyncState), ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(mism, 0, sizeof(unsigned), ctx->stream);
    auto run = [&](int r) -> hipError_t {
        switch (kind) {
            case SYNC_FLAT_FENCED: return launch_bench<SYNC_FLAT_FENCED>(s, slots, r, mism, nwg, ctx->stream);
            case SYNC_FLAT_DIRECT: return launch_bench<SYNC_FLAT_DIRECT>(s, slots, r, mism, nwg, ctx->stream);
            case SYNC_XCD_DIRECT: return launch_bench<SYNC_XCD_DIRECT>(s, slots, r, mism, nwg, ctx->stream);
            default: return launch_bench<SYNC_XCD_FLAGS>(s, slots, r, mism, nwg, ctx->stream);
        }
    };
    // a short launch first (code load, clocks), then the timed one; the
    // counters are reset between them so generations start at 1
    if (e == hipSuccess) e = run(2);
    if (e == hipSuccess) e = hipMemsetAsync(s, 0, sizeof(SyncState), ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(ctx->t0, ctx->stream);
    if (e == hipSuccess) e = run(rounds);
    if (e == hipSuccess) e = hipEventRecord(ctx->t1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(ctx->t1);
    float ms = 0.0f;
    unsigned m = 0, err[1] = {0};
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ctx->t0, ctx->t1);
    if (e == hipSuccess) e = hipMemcpy(&m, mism, sizeof(unsigned), hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(err, s->err, sizeof(unsigned), hipMemcpyDeviceToHost);
    if (s) (void)hipFree(s);
    if (slots) (void)hipFree(slots);
    if (mism) (void)hipFree(mism);
    if (e == hipErrorCooperativeLaunchTooLarge) return fail(LQ8_ERR_INVALID_ARG, "grid too large to be co-resident");
    if (e != hipSuccess) return hip_fail(e, "grid sync benchmark");
    *us_per_sync = ms * 1000.0f / (2.0f * rounds);
    *mismatches = m;
    *gave_up = err[0];
    return LQ8_OK;
}
