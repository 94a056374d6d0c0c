// runtime.hip -- context, weights, linear forward: the C ABI of include/lq8.h
// (model entry points live in model.hip).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <unordered_set>
#include <vector>

#include "lq8_internal.h"

namespace lq8 {

namespace {
thread_local std::string g_last_error;
std::mutex g_reg_mu;
std::unordered_set<const void*>& registry() {
    static std::unordered_set<const void*> s;
    return s;
}
}  // namespace

void set_error(const std::string& msg) { g_last_error = msg; }

lq8_status fail(lq8_status st, const std::string& msg) {
    g_last_error = msg;
    return st;
}

lq8_status hip_fail(hipError_t e, const char* what) {
    std::string m = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    if (e == hipErrorOutOfMemory) return fail(LQ8_ERR_OUT_OF_MEMORY, m);
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) return fail(LQ8_ERR_NO_DEVICE, m);
    return fail(LQ8_ERR_DEVICE, m);
}

void registry_add(const void* p) {
    std::lock_guard<std::mutex> g(g_reg_mu);
    registry().insert(p);
}
void registry_remove(const void* p) {
    std::lock_guard<std::mutex> g(g_reg_mu);
    registry().erase(p);
}
bool registry_has(const void* p) {
    std::lock_guard<std::mutex> g(g_reg_mu);
    return p && registry().count(p) != 0;
}

lq8_status ctx_scratch(lq8_ctx* ctx, size_t bytes, void** out) {
    if (bytes > ctx->scratch_bytes) {
        LQ8_HIP(hipStreamSynchronize(ctx->stream));
        if (ctx->scratch) LQ8_HIP(hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        LQ8_HIP(hipMalloc(&ctx->scratch, want));
        ctx->scratch_bytes = want;
    }
    *out = ctx->scratch;
    return LQ8_OK;
}

lq8_status weight_alloc(lq8_ctx* ctx, size_t n_out, size_t k_in, lq8_weight** out) {
    if (n_out == 0 || k_in == 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "weight: zero dimension");
    if (k_in % QK) return fail(LQ8_ERR_SHAPE_MISMATCH, "weight: k_in must be a multiple of 32 (Q8_0 block)");
    if (n_out > (size_t)INT32_MAX || k_in > (size_t)INT32_MAX) return fail(LQ8_ERR_SHAPE_MISMATCH, "weight: too large");
    lq8_weight* w = new lq8_weight();
    w->ctx = ctx;
    w->n_out = n_out;
    w->k_in = k_in;
    w->nb = k_in / QK;
    w->np = (w->nb + 1) / 2;
    w->tiles = (n_out + TILE_ROWS - 1) / TILE_ROWS;
    // storage rounds the rows up to 32 (two tiles): a 32-row MFMA operand never reads past it
    const size_t alloc_tiles = (n_out + 31) / 32 * 2;
    const size_t code_bytes = alloc_tiles * w->np * CHUNK_BYTES;
    const size_t scale_bytes = alloc_tiles * 2 * w->np * TILE_ROWS * sizeof(uint16_t);
    hipError_t e = hipMalloc(&w->codes, code_bytes);
    if (e == hipSuccess) e = hipMalloc(&w->scales, scale_bytes);
    // padding rows and the padding block of an odd nb are zero
    if (e == hipSuccess) e = hipMemsetAsync(w->codes, 0, code_bytes, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(w->scales, 0, scale_bytes, ctx->stream);
    if (e != hipSuccess) {
        weight_release(w);
        return hip_fail(e, "weight allocation");
    }
    registry_add(w);
    *out = w;
    return LQ8_OK;
}

void weight_release(lq8_weight* w) {
    if (!w) return;
    registry_remove(w);
    if (w->codes) (void)hipFree(w->codes);
    if (w->scales) (void)hipFree(w->scales);
    delete w;
}

// ---- host Q8_0 quantizer (same algorithm as the device quantizer) ---------

static inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

uint16_t host_f32_to_f16(float f) {
    uint32_t x = f2u(f), sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u | ((ax >> 13) & 0x3FFu) : 0x7C00u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax >= 0x38800000u) {
        uint32_t m = ax & 0x7FFFFFu, h = (((ax >> 23) - 112u) << 10) | (m >> 13), rem = m & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    int s = 126 - (int)(ax >> 23);
    uint32_t h = m >> s, rem = m & ((1u << s) - 1u), half = 1u << (s - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float host_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

}  // namespace lq8

using namespace lq8;

#define CHECK_CTX(ctx) \
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid or released context handle")
#define CHECK_W(w) \
    if (!registry_has(w)) return fail(LQ8_ERR_INVALID_ARG, "invalid or released weight handle")

static lq8_status set_device(lq8_ctx* ctx) {
    LQ8_HIP(hipSetDevice(ctx->device));
    return LQ8_OK;
}

// ---- scratch of the allocation-free linear forward ---------------------------
// lq8_linear_forward_device_noalloc quantizes its activation rows into this
// file-scope device array instead of context memory: one copy per GPU, held
// until the process ends, shared by every call on that GPU (calls that
// overlap on one GPU race).  Host code never hands `scratch` itself to a
// kernel -- in host code the name is a stand-in, not a device address: each
// device's copy is resolved once by hipGetSymbolAddress at lq8_init (with
// that device current) and only that address is used.
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)8 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};  // per device: the address of its copy of `scratch`
}  // namespace

// With `device` current: resolve its copy of the scratch array once.
static lq8_status resolve_scratch(int device) {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (device < 0 || device >= MAX_DEVICES) return fail(LQ8_ERR_NO_DEVICE, "device index above 63");
    if (g_scratch_ptr[device]) return LQ8_OK;
    void* p = nullptr;
    LQ8_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(LQ8_ERR_DEVICE, "scratch: no device address");
    g_scratch_ptr[device] = p;
    return LQ8_OK;
}

static void* device_scratch(int device) {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    return device >= 0 && device < MAX_DEVICES ? g_scratch_ptr[device] : nullptr;
}

extern "C" {

const char* lq8_version(void) { return "lq8 0.1.0 (gfx950, Q8_0)"; }

const char* lq8_last_error(void) { return g_last_error.c_str(); }

lq8_status lq8_device_count(int* count) {
    if (!count) return fail(LQ8_ERR_INVALID_ARG, "count is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return LQ8_OK;
}

size_t lq8_q8_0_bytes(size_t n) { return (n / QK) * BLOCK_BYTES; }

lq8_status lq8_quantize_q8_0(const float* x, size_t n, void* blocks_out) {
    if ((!x || !blocks_out) && n) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (n % QK) return fail(LQ8_ERR_SHAPE_MISMATCH, "quantize: n must be a multiple of 32");
    uint8_t* o = (uint8_t*)blocks_out;
    for (size_t b = 0; b < n / QK; b++) {
        const float* xb = x + b * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; j++) {
            float v = std::fabs(xb[j]);
            if (v > amax) amax = v;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t d16 = host_f32_to_f16(d);
        uint8_t* ob = o + b * BLOCK_BYTES;
        ob[0] = (uint8_t)(d16 & 0xFF);
        ob[1] = (uint8_t)(d16 >> 8);
        for (int j = 0; j < QK; j++) {
            float v = std::round(xb[j] * id);
            int q = (v != v) ? 0 : (v >= 127.0f ? 127 : (v <= -128.0f ? -128 : (int)v));
            ob[2 + j] = (uint8_t)(int8_t)q;
        }
    }
    return LQ8_OK;
}

lq8_status lq8_dequantize_q8_0(const void* blocks, size_t n, float* y) {
    if ((!blocks || !y) && n) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (n % QK) return fail(LQ8_ERR_SHAPE_MISMATCH, "dequantize: n must be a multiple of 32");
    const uint8_t* in = (const uint8_t*)blocks;
    for (size_t b = 0; b < n / QK; b++) {
        const uint8_t* blk = in + b * BLOCK_BYTES;
        float d = host_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < QK; j++) y[b * QK + j] = d * (float)(int8_t)blk[2 + j];
    }
    return LQ8_OK;
}

lq8_status lq8_init(int device, lq8_ctx** out) {
    if (!out) return fail(LQ8_ERR_INVALID_ARG, "out is null");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(LQ8_ERR_NO_DEVICE, "no HIP device available (no fallback: the Q8_0 path requires a GPU)");
    if (device < 0 || device >= n) return fail(LQ8_ERR_NO_DEVICE, "device index out of range");
    LQ8_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    LQ8_HIP(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(LQ8_ERR_NO_DEVICE, std::string("device is ") + prop.gcnArchName + ", this library targets gfx950");
    lq8_status st = resolve_scratch(device);
    if (st) return st;
    lq8_ctx* ctx = new lq8_ctx();
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreate(&ctx->t0);
    if (e == hipSuccess) e = hipEventCreate(&ctx->t1);
    if (e != hipSuccess) {
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_fail(e, "context creation");
    }
    registry_add(ctx);
    *out = ctx;
    return LQ8_OK;
}

lq8_status lq8_shutdown(lq8_ctx* ctx) {
    CHECK_CTX(ctx);
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    registry_remove(ctx);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->problems) (void)hipFree(ctx->problems);
    if (ctx->io_dev) (void)hipFree(ctx->io_dev);
    if (ctx->io_host) (void)hipHostFree(ctx->io_host);
    (void)hipEventDestroy(ctx->t0);
    (void)hipEventDestroy(ctx->t1);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return LQ8_OK;
}

lq8_status lq8_synchronize(lq8_ctx* ctx) {
    CHECK_CTX(ctx);
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    return LQ8_OK;
}

lq8_status lq8_device_alloc(lq8_ctx* ctx, size_t bytes, void** dptr) {
    CHECK_CTX(ctx);
    if (!dptr) return fail(LQ8_ERR_INVALID_ARG, "dptr is null");
    if (set_device(ctx)) return LQ8_ERR_DEVICE;
    LQ8_HIP(hipMalloc(dptr, bytes ? bytes : 1));
    return LQ8_OK;
}

lq8_status lq8_device_free(lq8_ctx* ctx, void* dptr) {
    CHECK_CTX(ctx);
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    LQ8_HIP(hipFree(dptr));
    return LQ8_OK;
}

lq8_status lq8_copy_to_device(lq8_ctx* ctx, void* dst, const void* src, size_t bytes) {
    CHECK_CTX(ctx);
    LQ8_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    return LQ8_OK;
}

lq8_status lq8_copy_to_host(lq8_ctx* ctx, void* dst, const void* src, size_t bytes) {
    CHECK_CTX(ctx);
    LQ8_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    return LQ8_OK;
}

lq8_status lq8_copy_device(lq8_ctx* ctx, void* dst, const void* src, size_t bytes) {
    CHECK_CTX(ctx);
    if ((!dst || !src) && bytes) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (!bytes) return LQ8_OK;
    LQ8_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return LQ8_OK;
}

lq8_status lq8_timer_start(lq8_ctx* ctx) {
    CHECK_CTX(ctx);
    LQ8_HIP(hipEventRecord(ctx->t0, ctx->stream));
    return LQ8_OK;
}

lq8_status lq8_timer_stop(lq8_ctx* ctx, float* elapsed_ms) {
    CHECK_CTX(ctx);
    if (!elapsed_ms) return fail(LQ8_ERR_INVALID_ARG, "elapsed_ms is null");
    LQ8_HIP(hipEventRecord(ctx->t1, ctx->stream));
    LQ8_HIP(hipEventSynchronize(ctx->t1));
    LQ8_HIP(hipEventElapsedTime(elapsed_ms, ctx->t0, ctx->t1));
    return LQ8_OK;
}

// ---- weights -------------------------------------------------------------------

lq8_status lq8_weight_upload(lq8_ctx* ctx, const void* blocks, size_t n_out, size_t k_in, lq8_weight** out) {
    CHECK_CTX(ctx);
    if (!blocks || !out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (set_device(ctx)) return LQ8_ERR_DEVICE;
    lq8_weight* w = nullptr;
    lq8_status st = weight_alloc(ctx, n_out, k_in, &w);
    if (st) return st;
    size_t bytes = n_out * (k_in / QK) * BLOCK_BYTES;
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, bytes);
    if (e == hipSuccess) e = hipMemcpyAsync(tmp, blocks, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) {
        if (tmp) (void)hipFree(tmp);
        weight_release(w);
        return hip_fail(e, "weight upload");
    }
    st = launch_repack_aos(ctx->stream, (const uint8_t*)tmp, n_out, 0, w);
    e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);
    if (st || e != hipSuccess) {
        weight_release(w);
        return st ? st : hip_fail(e, "weight repack");
    }
    *out = w;
    return LQ8_OK;
}

lq8_status lq8_weight_quantize_upload(lq8_ctx* ctx, const float* src, size_t n_out, size_t k_in, lq8_weight** out) {
    CHECK_CTX(ctx);
    if (!src || !out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (set_device(ctx)) return LQ8_ERR_DEVICE;
    lq8_weight* w = nullptr;
    lq8_status st = weight_alloc(ctx, n_out, k_in, &w);
    if (st) return st;
    size_t bytes = n_out * k_in * sizeof(float);
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, bytes);
    if (e == hipSuccess) e = hipMemcpyAsync(tmp, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) {
        if (tmp) (void)hipFree(tmp);
        weight_release(w);
        return hip_fail(e, "weight upload");
    }
    st = launch_quantize_weight_f32(ctx->stream, (const float*)tmp, n_out, 0, w);
    e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);
    if (st || e != hipSuccess) {
        weight_release(w);
        return st ? st : hip_fail(e, "weight quantize");
    }
    *out = w;
    return LQ8_OK;
}

lq8_status lq8_weight_quantize_upload_bf16(lq8_ctx* ctx, const uint16_t* src, size_t n_out, size_t k_in,
                                           lq8_weight** out) {
    CHECK_CTX(ctx);
    if (!src || !out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (set_device(ctx)) return LQ8_ERR_DEVICE;
    lq8_weight* w = nullptr;
    lq8_status st = weight_alloc(ctx, n_out, k_in, &w);
    if (st) return st;
    const size_t bytes = n_out * k_in * sizeof(uint16_t);
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, bytes);
    if (e == hipSuccess) e = hipMemcpyAsync(tmp, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) {
        if (tmp) (void)hipFree(tmp);
        weight_release(w);
        return hip_fail(e, "weight upload");
    }
    st = launch_quantize_weight_bf16(ctx->stream, (const uint16_t*)tmp, n_out, 0, w);
    e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);
    if (st || e != hipSuccess) {
        weight_release(w);
        return st ? st : hip_fail(e, "weight quantize");
    }
    *out = w;
    return LQ8_OK;
}

lq8_status lq8_weight_random(lq8_ctx* ctx, size_t n_out, size_t k_in, uint64_t seed, uint64_t stream, float stddev,
                             lq8_weight** out) {
    CHECK_CTX(ctx);
    if (!out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (set_device(ctx)) return LQ8_ERR_DEVICE;
    lq8_weight* w = nullptr;
    lq8_status st = weight_alloc(ctx, n_out, k_in, &w);
    if (st) return st;
    st = launch_random_weight(ctx->stream, w, 0, n_out, seed, stream, stddev);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (st || e != hipSuccess) {
        weight_release(w);
        return st ? st : hip_fail(e, "random weight");
    }
    *out = w;
    return LQ8_OK;
}

lq8_status lq8_weight_download(lq8_ctx* ctx, const lq8_weight* w, void* blocks_out) {
    CHECK_CTX(ctx);
    CHECK_W(w);
    if (!blocks_out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    size_t bytes = w->n_out * w->nb * BLOCK_BYTES;
    void* tmp = nullptr;
    LQ8_HIP(hipMalloc(&tmp, bytes));
    lq8_status st = launch_unpack_aos(ctx->stream, w, 0, w->n_out, (uint8_t*)tmp);
    hipError_t e = st ? hipSuccess : hipMemcpyAsync(blocks_out, tmp, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);
    if (st) return st;
    if (e != hipSuccess) return hip_fail(e, "weight download");
    return LQ8_OK;
}

lq8_status lq8_weight_shape(const lq8_weight* w, size_t* n_out, size_t* k_in) {
    CHECK_W(w);
    if (n_out) *n_out = w->n_out;
    if (k_in) *k_in = w->k_in;
    return LQ8_OK;
}

lq8_status lq8_weight_free(lq8_weight* w) {
    CHECK_W(w);
    (void)hipStreamSynchronize(w->ctx->stream);
    weight_release(w);
    return LQ8_OK;
}

lq8_status lq8_quantize_q8_0_device(lq8_ctx* ctx, const float* d_x, size_t n, void* d_blocks) {
    CHECK_CTX(ctx);
    if ((!d_x || !d_blocks) && n) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (n % QK) return fail(LQ8_ERR_SHAPE_MISMATCH, "quantize: n must be a multiple of 32");
    return launch_quantize_aos(ctx->stream, d_x, n / QK, (uint8_t*)d_blocks);
}

lq8_status lq8_quantize_activations_device(lq8_ctx* ctx, int source, const float* d_x, const float* d_w, size_t m,
                                          size_t k, float eps, void* d_blocks) {
    CHECK_CTX(ctx);
    if (!d_x || !d_blocks || (source == LQ8_ACT_RMSNORM && !d_w)) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (source < LQ8_ACT_PLAIN || source > LQ8_ACT_SILU_MUL) return fail(LQ8_ERR_INVALID_ARG, "unknown activation source");
    if (k == 0 || k % QK || k > (size_t)INT32_MAX / 4) return fail(LQ8_ERR_SHAPE_MISMATCH, "k must be a positive multiple of 32");
    if (m == 0) return LQ8_OK;
    if (m > (size_t)INT32_MAX / 2) return fail(LQ8_ERR_SHAPE_MISMATCH, "m too large");
    if (((uintptr_t)d_x & 15) != 0) return fail(LQ8_ERR_INVALID_ARG, "x must be 16-byte aligned");
    const int mi = (int)m, ki = (int)k;
    const size_t cb = act_code_bytes(mi, ki), sb = act_scale_bytes(mi, ki);
    // RmsNorm rows wider than the fused kernel handles go through normed rows first (the prefill path)
    const bool two_step = source == LQ8_ACT_RMSNORM && !rms_quantize_supported(ki);
    const size_t rows_bytes = two_step ? m * k * sizeof(float) : 0;
    void* sc = nullptr;
    lq8_status st = ctx_scratch(ctx, cb + sb + rows_bytes, &sc);
    if (st) return st;
    int8_t* xq = (int8_t*)sc;
    uint32_t* xs = (uint32_t*)((char*)sc + cb);
    if (source == LQ8_ACT_PLAIN) {
        st = launch_quantize_act(ctx->stream, d_x, mi, ki, xq, xs);
    } else if (source == LQ8_ACT_SILU_MUL) {
        st = launch_silu_quantize_act(ctx->stream, d_x, mi, ki, xq, xs);
    } else if (two_step) {
        float* rows = (float*)((char*)sc + cb + sb);
        st = launch_rms_norm_rows(ctx->stream, d_x, d_w, mi, ki, eps, rows);
        if (!st) st = launch_quantize_act(ctx->stream, rows, mi, ki, xq, xs);
    } else {
        st = launch_rms_quantize_act(ctx->stream, d_x, d_w, mi, ki, eps, xq, xs);
    }
    if (st) return st;
    return launch_unpack_act(ctx->stream, xq, xs, mi, ki, (uint8_t*)d_blocks);
}

lq8_status lq8_weight_dequantize_rows_device(lq8_ctx* ctx, const lq8_weight* w, size_t row0, size_t nrows,
                                             float* d_y) {
    CHECK_CTX(ctx);
    CHECK_W(w);
    if (!d_y) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (row0 > w->n_out || nrows > w->n_out - row0) return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "rows out of range");
    return launch_dequant_rows(ctx->stream, w, nullptr, row0, nrows, d_y);
}

// ---- decoder ops ------------------------------------------------------------------

lq8_status lq8_rms_norm_device(lq8_ctx* ctx, const float* d_x, const float* d_w, size_t rows, size_t dim, float eps,
                               float* d_y) {
    CHECK_CTX(ctx);
    if (!d_x || !d_w || !d_y) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (dim == 0 || dim > (size_t)INT32_MAX || rows > 0x7FFFFFFF) return fail(LQ8_ERR_SHAPE_MISMATCH, "bad shape");
    if (rows == 0) return LQ8_OK;
    return launch_rms_norm_rows(ctx->stream, d_x, d_w, (int)rows, (int)dim, eps, d_y);
}

lq8_status lq8_silu_device(lq8_ctx* ctx, const float* d_x, size_t n, float* d_y) {
    CHECK_CTX(ctx);
    if ((!d_x || !d_y) && n) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    return launch_silu(ctx->stream, d_x, n, d_y);
}

// ---- linear forward --------------------------------------------------------------

lq8_status lq8_gemv_q8_0_device(lq8_ctx* ctx, const lq8_weight* w, const float* d_x, float* d_y) {
    CHECK_CTX(ctx);
    CHECK_W(w);
    if (!d_x || !d_y) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (((uintptr_t)d_x & 15) != 0) return fail(LQ8_ERR_INVALID_ARG, "x must be 16-byte aligned");
    GemvArgs a{w->codes, w->scales, d_x, nullptr, d_y, nullptr, nullptr, nullptr, (int)w->n_out, (int)w->k_in, 0.0f};
    return launch_gemv(ctx->stream, XS_PLAIN, EPI_STORE, a);
}

lq8_status lq8_gemm_q8_0_device(lq8_ctx* ctx, const lq8_weight* w, const float* d_x, size_t m, float* d_y) {
    CHECK_CTX(ctx);
    CHECK_W(w);
    if (!d_x || !d_y) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (m == 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemm: m must be positive");
    if (m > (size_t)INT32_MAX / 2) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemm: m too large");
    if (((uintptr_t)d_x & 15) != 0) return fail(LQ8_ERR_INVALID_ARG, "x must be 16-byte aligned");
    const size_t code_bytes = act_code_bytes((int)m, (int)w->k_in), scale_bytes = act_scale_bytes((int)m, (int)w->k_in);
    void* sc = nullptr;
    lq8_status st = ctx_scratch(ctx, code_bytes + scale_bytes, &sc);
    if (st) return st;
    int8_t* xq = (int8_t*)sc;
    uint32_t* xs = (uint32_t*)((char*)sc + code_bytes);
    st = launch_quantize_act(ctx->stream, d_x, (int)m, (int)w->k_in, xq, xs);
    if (st) return st;
    return launch_gemm(ctx->stream, xq, xs, (int)m, w, d_y, nullptr);
}

lq8_status lq8_linear_forward_device(lq8_ctx* ctx, const lq8_weight* w, const float* d_x, size_t m, float* d_y) {
    if (m == 1) return lq8_gemv_q8_0_device(ctx, w, d_x, d_y);
    return lq8_gemm_q8_0_device(ctx, w, d_x, m, d_y);
}

lq8_status lq8_linear_forward_device_noalloc(lq8_ctx* ctx, const lq8_weight* w, const float* d_x, size_t m,
                                             float* d_y) {
    CHECK_CTX(ctx);
    CHECK_W(w);
    if (!d_x || !d_y) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (m == 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "linear: m must be positive");
    if (((uintptr_t)d_x & 15) != 0) return fail(LQ8_ERR_INVALID_ARG, "x must be 16-byte aligned");
    if (m == 1) return lq8_gemv_q8_0_device(ctx, w, d_x, d_y);  // the GEMV needs no scratch
    if (m > (size_t)INT32_MAX / 2) return fail(LQ8_ERR_SHAPE_MISMATCH, "linear: m too large");
    const size_t cb = act_code_bytes((int)m, (int)w->k_in), sb = act_scale_bytes((int)m, (int)w->k_in);
    if (cb + sb > NOALLOC_SCRATCH_BYTES)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "linear (no allocation): the activation operand of " + std::to_string(m) +
                                                " x " + std::to_string(w->k_in) + " needs " + std::to_string(cb + sb) +
                                                " bytes, above the 8 MiB static scratch");
    char* base = (char*)device_scratch(ctx->device);
    if (!base) return fail(LQ8_ERR_DEVICE, "scratch: not resolved for this device");
    // the quantizer writes every code and scale the GEMM reads (zeros in the
    // padding), so nothing in the array has to be cleared between calls
    int8_t* xq = (int8_t*)base;
    uint32_t* xs = (uint32_t*)(base + cb);
    lq8_status st = launch_quantize_act(ctx->stream, d_x, (int)m, (int)w->k_in, xq, xs);
    if (st) return st;
    return launch_gemm(ctx->stream, xq, xs, (int)m, w, d_y, nullptr);
}

namespace {
// n16 16-byte words from src to dst, one workgroup (the GEMV's input, 4-48
// KiB, out of the mapped pinned staging: one PCIe round trip per load batch).
__global__ __launch_bounds__(1024) void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n16) {
    constexpr int U = 4;
    for (size_t i0 = threadIdx.x; i0 < n16; i0 += 1024 * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = i0 + u * 1024 < n16 ? src[i0 + u * 1024] : uint4{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < U; u++)
            if (i0 + u * 1024 < n16) dst[i0 + u * 1024] = v[u];
    }
}
}  // namespace

// Device and pinned host staging for the host-pointer entry points: grows
// (after a synchronize) only when a call needs more than any call before.
static lq8_status ctx_io(lq8_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->io_bytes) return LQ8_OK;
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->io_dev) LQ8_HIP(hipFree(ctx->io_dev));
    if (ctx->io_host) LQ8_HIP(hipHostFree(ctx->io_host));
    ctx->io_dev = ctx->io_host = ctx->io_host_dev = nullptr;
    ctx->io_bytes = 0;
    const size_t want = std::max(bytes, (size_t)1 << 20);
    LQ8_HIP(hipMalloc(&ctx->io_dev, want));
    LQ8_HIP(hipHostMalloc(&ctx->io_host, want, hipHostMallocDefault));
    LQ8_HIP(hipHostGetDevicePointer(&ctx->io_host_dev, ctx->io_host, 0));
    ctx->io_bytes = want;
    return LQ8_OK;
}

lq8_status lq8_linear_forward(lq8_ctx* ctx, const lq8_weight* w, const float* x, size_t m, float* y) {
    CHECK_CTX(ctx);
    CHECK_W(w);
    if (!x || !y) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (m == 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "linear: m must be positive");
    if (set_device(ctx)) return LQ8_ERR_DEVICE;
    // x at offset 0, y after it (256-byte aligned), in the context's staging:
    // host x -> pinned -> HBM, the device forward, HBM -> pinned -> host y
    const size_t xb = m * w->k_in * sizeof(float), yb = m * w->n_out * sizeof(float);
    const size_t yoff = (xb + 255) & ~(size_t)255;
    lq8_status st = ctx_io(ctx, yoff + yb);
    if (st) return st;
    char* dio = (char*)ctx->io_dev;
    char* hio = (char*)ctx->io_host;
    std::memcpy(hio, x, xb);
    if (m == 1) {
        // one vector: a one-workgroup kernel copies x out of the mapped pinned
        // buffer and the GEMV stores y into it (no copy engine between the
        // compute queue's steps)
        char* hdev = (char*)ctx->io_host_dev;
        hipLaunchKernelGGL(k_copy16, dim3(1), dim3(1024), 0, ctx->stream, (const uint4*)hdev, (uint4*)dio, xb / 16);
        LQ8_HIP(hipGetLastError());
        st = lq8_gemv_q8_0_device(ctx, w, (const float*)dio, (float*)(hdev + yoff));
    } else {
        LQ8_HIP(hipMemcpyAsync(dio, hio, xb, hipMemcpyHostToDevice, ctx->stream));
        st = lq8_linear_forward_device(ctx, w, (const float*)dio, m, (float*)(dio + yoff));
        if (!st) LQ8_HIP(hipMemcpyAsync(hio + yoff, dio + yoff, yb, hipMemcpyDeviceToHost, ctx->stream));
    }
    if (st) {
        (void)hipStreamSynchronize(ctx->stream);
        return st;
    }
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    std::memcpy(y, hio + yoff, yb);
    return LQ8_OK;
}

lq8_status lq8_gemv_grouped_device(lq8_ctx* ctx, const lq8_gemv_problem* problems, size_t count) {
    CHECK_CTX(ctx);
    if (count == 0) return LQ8_OK;
    if (!problems) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (count > 65536) return fail(LQ8_ERR_INVALID_ARG, "too many problems");
    std::vector<GemvProblemDev> host(count);
    size_t tiles = 0;
    int max_k = 0;
    for (size_t i = 0; i < count; i++) {
        const lq8_gemv_problem& p = problems[i];
        if (!registry_has(p.w)) return fail(LQ8_ERR_INVALID_ARG, "invalid weight handle in problem list");
        if (!p.x || !p.y) return fail(LQ8_ERR_INVALID_ARG, "null pointer in problem list");
        if (((uintptr_t)p.x & 15) != 0) return fail(LQ8_ERR_INVALID_ARG, "x must be 16-byte aligned");
        if (p.w->k_in > (size_t)GEMV_MAX_K) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k above 12288 is not supported");
        host[i] = GemvProblemDev{p.w->codes, p.w->scales, p.x, p.y, (int)p.w->n_out, (int)p.w->k_in, (int)tiles, 0};
        tiles += p.w->tiles;
        if ((int)p.w->k_in > max_k) max_k = (int)p.w->k_in;
    }
    if (tiles > (size_t)INT32_MAX) return fail(LQ8_ERR_SHAPE_MISMATCH, "too many tiles");
    size_t bytes = count * sizeof(GemvProblemDev);
    if (bytes > ctx->problems_bytes) {
        LQ8_HIP(hipStreamSynchronize(ctx->stream));
        if (ctx->problems) LQ8_HIP(hipFree(ctx->problems));
        ctx->problems = nullptr;
        LQ8_HIP(hipMalloc(&ctx->problems, bytes));
        ctx->problems_bytes = bytes;
    }
    LQ8_HIP(hipMemcpyAsync(ctx->problems, host.data(), bytes, hipMemcpyHostToDevice, ctx->stream));
    // the host vector dies at return: wait for the copy to finish reading it
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    return launch_gemv_grouped(ctx->stream, (const GemvProblemDev*)ctx->problems, (int)count, (int)tiles, max_k);
}

lq8_status lq8_bench_gemv(lq8_ctx* ctx, const lq8_gemv_problem* problems, size_t count, int mode, int reps,
                          float* ms) {
    CHECK_CTX(ctx);
    if (!problems || !count || reps <= 0 || !ms) return fail(LQ8_ERR_INVALID_ARG, "bad benchmark arguments");
    std::vector<GemvArgs> L(count);
    for (size_t i = 0; i < count; i++) {
        const lq8_gemv_problem& p = problems[i];
        if (!registry_has(p.w)) return fail(LQ8_ERR_INVALID_ARG, "invalid weight handle in problem list");
        if (!p.x || !p.y || ((uintptr_t)p.x & 15)) return fail(LQ8_ERR_INVALID_ARG, "bad x / y pointer");
        if (p.w->k_in > (size_t)GEMV_MAX_K) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k above 12288 is not supported");
        L[i] = GemvArgs{p.w->codes, p.w->scales, p.x, nullptr, p.y, nullptr, nullptr, nullptr, (int)p.w->n_out,
                        (int)p.w->k_in, 0.0f};
    }
    hipStream_t s = ctx->stream;
    lq8_status st = LQ8_OK;
    if (mode == 0 || mode == 2) {  // one launch per problem (2: replayed as a HIP graph)
        hipGraphExec_t exec = nullptr;
        if (mode == 2) {
            hipGraph_t g = nullptr;
            LQ8_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
            for (size_t i = 0; i < count && !st; i++) st = launch_gemv(s, XS_PLAIN, EPI_STORE, L[i]);
            hipError_t e = hipStreamEndCapture(s, &g);
            if (st) { if (g) (void)hipGraphDestroy(g); return st; }
            if (e != hipSuccess) return hip_fail(e, "capture");
            e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (e != hipSuccess) return hip_fail(e, "instantiate");
        }
        LQ8_HIP(hipEventRecord(ctx->t0, s));
        for (int r = 0; r < reps && !st; r++) {
            if (exec) {
                hipError_t e = hipGraphLaunch(exec, s);
                if (e != hipSuccess) st = hip_fail(e, "graph launch");
            } else {
                for (size_t i = 0; i < count && !st; i++) st = launch_gemv(s, XS_PLAIN, EPI_STORE, L[i]);
            }
        }
        LQ8_HIP(hipEventRecord(ctx->t1, s));
        LQ8_HIP(hipEventSynchronize(ctx->t1));
        if (exec) (void)hipGraphExecDestroy(exec);
        if (st) return st;
        LQ8_HIP(hipEventElapsedTime(ms, ctx->t0, ctx->t1));
        return LQ8_OK;
    }
    if (mode == 1) {  // all problems in one grouped launch
        std::vector<GemvProblemDev> host(count);
        size_t tiles = 0;
        int max_k = 0;
        for (size_t i = 0; i < count; i++) {
            const lq8_gemv_problem& p = problems[i];
            host[i] = GemvProblemDev{p.w->codes, p.w->scales, p.x, p.y, (int)p.w->n_out, (int)p.w->k_in, (int)tiles, 0};
            tiles += p.w->tiles;
            max_k = std::max(max_k, (int)p.w->k_in);
        }
        size_t bytes = count * sizeof(GemvProblemDev);
        void* d = nullptr;
        LQ8_HIP(hipMalloc(&d, bytes));
        hipError_t e = hipMemcpy(d, host.data(), bytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipEventRecord(ctx->t0, s);
        for (int r = 0; r < reps && e == hipSuccess && !st; r++)
            st = launch_gemv_grouped(s, (const GemvProblemDev*)d, (int)count, (int)tiles, max_k);
        if (e == hipSuccess) e = hipEventRecord(ctx->t1, s);
        if (e == hipSuccess) e = hipEventSynchronize(ctx->t1);
        (void)hipFree(d);
        if (st) return st;
        if (e != hipSuccess) return hip_fail(e, "grouped benchmark");
        LQ8_HIP(hipEventElapsedTime(ms, ctx->t0, ctx->t1));
        return LQ8_OK;
    }
    if (mode == 3) {  // per-launch event pairs: sum of the launches' own intervals
        std::vector<hipEvent_t> ev(2 * count);
        for (auto& e : ev) LQ8_HIP(hipEventCreate(&e));
        double total = 0.0;
        for (int r = 0; r < reps && !st; r++) {
            for (size_t i = 0; i < count && !st; i++) {
                (void)hipEventRecord(ev[2 * i], s);
                st = launch_gemv(s, XS_PLAIN, EPI_STORE, L[i]);
                (void)hipEventRecord(ev[2 * i + 1], s);
            }
            if (st) break;
            hipError_t e = hipEventSynchronize(ev[2 * count - 1]);
            if (e != hipSuccess) { st = hip_fail(e, "event sync"); break; }
            for (size_t i = 0; i < count; i++) {
                float t = 0;
                (void)hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]);
                total += t;
            }
        }
        for (auto& e : ev) (void)hipEventDestroy(e);
        if (st) return st;
        *ms = (float)total;
        return LQ8_OK;
    }
    return fail(LQ8_ERR_INVALID_ARG, "unknown benchmark mode");
}

}  // extern "C"
