// bench_floors.hip -- the hardware floors the latency-bound kernels of this
// library are measured against: the period of back-to-back launches of an
// empty kernel, the read-only streaming rate of the whole chip and of one
// compute unit, and the latency of one dependent load from HBM.
#include <algorithm>
#include <random>
#include <vector>

#include "lq8_internal.h"

namespace lq8 {

namespace {

constexpr int FLOOR_THREADS = 512;
constexpr int STREAM_UNROLL = 8;  // 16-byte loads in flight per thread
typedef unsigned v4u __attribute__((ext_vector_type(4)));

__global__ void k_empty() {}

// Reads n16 16-byte words, STREAM_UNROLL independent loads per thread per
// round (nontemporal: the stream is read once).  The buffer is zero, so the
// store below never runs; it keeps the loads live.
__global__ __launch_bounds__(FLOOR_THREADS) void k_stream_read(const v4u* __restrict__ p, size_t n16,
                                                               unsigned* out) {
    const size_t stride = (size_t)gridDim.x * FLOOR_THREADS;
    unsigned acc = 0;
    for (size_t i0 = (size_t)blockIdx.x * FLOOR_THREADS + threadIdx.x; i0 < n16; i0 += stride * STREAM_UNROLL) {
        v4u v[STREAM_UNROLL];
#pragma unroll
        for (int u = 0; u < STREAM_UNROLL; u++) {
            const size_t i = i0 + (size_t)u * stride;
            v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : v4u{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < STREAM_UNROLL; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

// The same reads by contiguous ranges: workgroup w streams the w-th of
// gridDim.x equal ranges, 8 KiB per load instruction of the workgroup.
__global__ __launch_bounds__(FLOOR_THREADS) void k_stream_chunks(const v4u* __restrict__ p, size_t n16,
                                                                 unsigned* out) {
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t lo = (size_t)blockIdx.x * per, hi = lo + per < n16 ? lo + per : n16;
    unsigned acc = 0;
    for (size_t i0 = lo + threadIdx.x; i0 < hi; i0 += (size_t)FLOOR_THREADS * STREAM_UNROLL) {
        v4u v[STREAM_UNROLL];
#pragma unroll
        for (int u = 0; u < STREAM_UNROLL; u++) {
            const size_t i = i0 + (size_t)u * FLOOR_THREADS;
            v[u] = i < hi ? __builtin_nontemporal_load(p + i) : v4u{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < STREAM_UNROLL; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}

// One thread follows `hops` links of a random cycle through the buffer: each
// load's address is the previous load's value, so every load waits for the
// last one's full round trip.
__global__ void k_chase(const uint32_t* __restrict__ next, int hops, uint32_t* out) {
    uint32_t i = 0;
    for (int h = 0; h < hops; h++) i = __builtin_nontemporal_load(next + i);
    out[0] = i;
}

}  // namespace

}  // namespace lq8

using namespace lq8;

extern "C" lq8_status lq8_bench_floors(lq8_ctx* ctx, int kind, int nwg, size_t bytes, int reps, double* value) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid context handle");
    if (!value) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (kind < LQ8_FLOOR_EMPTY || kind > LQ8_FLOOR_EMPTY_GRAPH) return fail(LQ8_ERR_INVALID_ARG, "unknown floor kind");
    if (nwg <= 0 || nwg > 65536 || reps <= 0 || reps > 1000000) return fail(LQ8_ERR_INVALID_ARG, "bad grid or repeat count");
    const bool empty = kind == LQ8_FLOOR_EMPTY || kind == LQ8_FLOOR_EMPTY_GRAPH;
    if (empty && (bytes != 0 && (bytes % 64 || bytes > 1024)))
        return fail(LQ8_ERR_INVALID_ARG, "empty kernel: bytes is the workgroup size (0: 64; a multiple of 64 up to 1024)");
    if (!empty && (bytes < 4096 || bytes > ((size_t)8 << 30) || bytes % 4096))
        return fail(LQ8_ERR_INVALID_ARG, "bytes must be a multiple of 4096 in [4 KiB, 8 GiB]");
    if (kind == LQ8_FLOOR_EMPTY_GRAPH && reps > 10000) return fail(LQ8_ERR_INVALID_ARG, "at most 10000 graph nodes");
    const unsigned wg_threads = empty && bytes ? (unsigned)bytes : 64u;
    LQ8_HIP(hipSetDevice(ctx->device));
    hipStream_t st = ctx->stream;
    void* buf = nullptr;
    unsigned* out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    lq8_status status = LQ8_OK;
    float ms = 0.0f;
    auto check = [&](hipError_t e, const char* what) {
        if (e != hipSuccess && status == LQ8_OK) status = hip_fail(e, what);
        return status == LQ8_OK;
    };
    if (check(hipEventCreate(&e0), "hipEventCreate") && check(hipEventCreate(&e1), "hipEventCreate") &&
        check(hipMalloc((void**)&out, 65536 * sizeof(unsigned)), "hipMalloc")) {
        if (kind == LQ8_FLOOR_EMPTY) {
            // reps back-to-back launches (one warm-up launch first)
            hipLaunchKernelGGL(k_empty, dim3((unsigned)nwg), dim3(wg_threads), 0, st);
            if (check(hipGetLastError(), "empty kernel") && check(hipEventRecord(e0, st), "hipEventRecord")) {
                for (int r = 0; r < reps && status == LQ8_OK; r++) {
                    hipLaunchKernelGGL(k_empty, dim3((unsigned)nwg), dim3(wg_threads), 0, st);
                    check(hipGetLastError(), "empty kernel");
                }
                if (check(hipEventRecord(e1, st), "hipEventRecord") && check(hipEventSynchronize(e1), "sync") &&
                    check(hipEventElapsedTime(&ms, e0, e1), "elapsed"))
                    *value = (double)ms * 1e3 / reps;  // us per launch
            }
        } else if (kind == LQ8_FLOOR_EMPTY_GRAPH) {
            // reps empty launches captured as one graph, replayed (once to warm up, then timed)
            hipGraph_t graph = nullptr;
            hipGraphExec_t exec = nullptr;
            if (check(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed), "capture")) {
                for (int r = 0; r < reps; r++) hipLaunchKernelGGL(k_empty, dim3((unsigned)nwg), dim3(wg_threads), 0, st);
                const hipError_t le = hipGetLastError();
                const hipError_t ce = hipStreamEndCapture(st, &graph);
                if (check(le, "empty kernel") && check(ce, "end capture") &&
                    check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate") &&
                    check(hipGraphLaunch(exec, st), "graph launch") && check(hipEventRecord(e0, st), "hipEventRecord") &&
                    check(hipGraphLaunch(exec, st), "graph launch") && check(hipEventRecord(e1, st), "hipEventRecord") &&
                    check(hipEventSynchronize(e1), "sync") && check(hipEventElapsedTime(&ms, e0, e1), "elapsed"))
                    *value = (double)ms * 1e3 / reps;  // us per graph node
            }
            if (exec) (void)hipGraphExecDestroy(exec);
            if (graph) (void)hipGraphDestroy(graph);
        } else if (kind == LQ8_FLOOR_STREAM || kind == LQ8_FLOOR_STREAM_CHUNKS) {
            if (check(hipMalloc(&buf, bytes), "hipMalloc") && check(hipMemsetAsync(buf, 0, bytes, st), "memset")) {
                const size_t n16 = bytes / 16;
                auto k = kind == LQ8_FLOOR_STREAM ? k_stream_read : k_stream_chunks;
                hipLaunchKernelGGL(k, dim3((unsigned)nwg), dim3(FLOOR_THREADS), 0, st, (const v4u*)buf, n16, out);
                if (check(hipGetLastError(), "stream kernel") && check(hipEventRecord(e0, st), "hipEventRecord")) {
                    for (int r = 0; r < reps && status == LQ8_OK; r++) {
                        hipLaunchKernelGGL(k, dim3((unsigned)nwg), dim3(FLOOR_THREADS), 0, st, (const v4u*)buf, n16,
                                           out);
                        check(hipGetLastError(), "stream kernel");
                    }
                    if (check(hipEventRecord(e1, st), "hipEventRecord") && check(hipEventSynchronize(e1), "sync") &&
                        check(hipEventElapsedTime(&ms, e0, e1), "elapsed"))
                        *value = (double)bytes * reps / ((double)ms * 1e-3) / 1e9;  // GB/s
                }
            }
        } else {
            // a random cycle through one 32-bit word per 128-byte line
            const size_t lines = bytes / 128, stride = 32;
            std::vector<uint32_t> order(lines);
            for (size_t i = 0; i < lines; i++) order[i] = (uint32_t)i;
            std::mt19937_64 rng(0x5EED);
            std::shuffle(order.begin() + 1, order.end(), rng);
            std::vector<uint32_t> next(lines * stride, 0);
            for (size_t i = 0; i < lines; i++) next[order[i] * stride] = (uint32_t)(order[(i + 1) % lines] * stride);
            if (check(hipMalloc(&buf, bytes), "hipMalloc") &&
                check(hipMemcpy(buf, next.data(), bytes, hipMemcpyHostToDevice), "copy")) {
                const int hops = std::min<int>(reps, (int)std::min<size_t>(lines, 1000000));
                hipLaunchKernelGGL(k_chase, dim3(1), dim3(1), 0, st, (const uint32_t*)buf, 64, out);
                if (check(hipGetLastError(), "chase kernel") && check(hipEventRecord(e0, st), "hipEventRecord")) {
                    hipLaunchKernelGGL(k_chase, dim3(1), dim3(1), 0, st, (const uint32_t*)buf, hops, out);
                    check(hipGetLastError(), "chase kernel");
                    if (check(hipEventRecord(e1, st), "hipEventRecord") && check(hipEventSynchronize(e1), "sync") &&
                        check(hipEventElapsedTime(&ms, e0, e1), "elapsed"))
                        *value = (double)ms * 1e6 / hops;  // ns per dependent load
                }
            }
        }
    }
    if (buf) (void)hipFree(buf);
    if (out) (void)hipFree(out);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    return status;
}
