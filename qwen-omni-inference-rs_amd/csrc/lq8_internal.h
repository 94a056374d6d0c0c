// lq8_internal.h -- shared definitions of the gfx950 Q8_0 library.
//
// Device layout of a Q8_0 weight W[n_out, k_in] (nb = k_in / 32 blocks per
// row, rows padded to a multiple of 64):
//   codes  [tiles = ceil(n_out/64)][nb][2 halves][64 rows][16 int8]
//   scales [tiles][nb][64 rows] f16 bits
// One (tile, block) pair is 2 KiB of codes: lane r of a wave reads row r's
// codes 0..15 from the first KiB and 16..31 from the second, so both 16-byte
// loads of a wave are 1 KiB contiguous.  The same layout feeds the MFMA GEMM
// (32-row halves of a tile are 512-byte contiguous operand slices).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/lq8.h"

namespace lq8 {

constexpr int QK = 32;
constexpr int BLOCK_BYTES = 34;
constexpr int TILE_ROWS = 64;
constexpr int GROUP_BLOCKS = 8;  // blocks per accumulation group
constexpr int TILE_BLOCK_BYTES = TILE_ROWS * QK;

// ---- error plumbing ------------------------------------------------------
void set_error(const std::string& msg);
lq8_status fail(lq8_status st, const std::string& msg);
lq8_status hip_fail(hipError_t e, const char* what);

#define LQ8_HIP(call)                                              \
    do {                                                           \
        hipError_t e_ = (call);                                    \
        if (e_ != hipSuccess) return ::lq8::hip_fail(e_, #call);   \
    } while (0)

// ---- handle registry (stale / foreign handles are rejected) ---------------
void registry_add(const void* p);
void registry_remove(const void* p);
bool registry_has(const void* p);

}  // namespace lq8

struct lq8_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    int num_cus = 0;
    // scratch for activation quantization (GEMM A operand) and staging
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    void* problems = nullptr;  // device copy of grouped GEMV descriptors
    size_t problems_bytes = 0;
};

struct lq8_weight {
    lq8_ctx* ctx = nullptr;
    size_t n_out = 0, k_in = 0, nb = 0, tiles = 0;
    int8_t* codes = nullptr;
    uint16_t* scales = nullptr;
};

namespace lq8 {

// Scratch owned by the context; grows on demand (synchronizes before growing).
lq8_status ctx_scratch(lq8_ctx* ctx, size_t bytes, void** out);

// ---- kernel launchers (kernels.hip) -------------------------------------
// x-source of a GEMV: plain f32 vector, RMSNorm of a hidden vector, or
// silu(gate) * up of a concatenated [gate | up] vector.
enum XSource : int { XS_PLAIN = 0, XS_RMSNORM = 1, XS_SILU = 2 };

struct GemvLaunch {
    const int8_t* codes;
    const uint16_t* scales;
    const float* x;        // XS_PLAIN: x[k]; XS_RMSNORM: hidden[k]; XS_SILU: gu[2k]
    const float* norm_w;   // XS_RMSNORM weight [k]
    float eps;
    float* y;              // output [n]
    const float* resid;    // if non-null: y = resid + Wx
    int n, k;
    // PARTIALS output: group partials [groups][stride] instead of y
    float* partials = nullptr;
    long long partials_cap = 0;
    // input as base + partials: x_i = (x ? x[i] : 0) + ((0 + xp[0][i]) + xp[1][i] + ...)
    const float* xp = nullptr;
    int xg = 0;
    size_t xstride = 0;
    float* x_out = nullptr;  // RMSNORM source: workgroup 0 stores the combined input here
};
lq8_status launch_gemv(hipStream_t s, XSource xs, const GemvLaunch& a);
// One workgroup per 64-row tile (all groups in one workgroup, no counters).
lq8_status launch_gemv_tile_wg(hipStream_t s, XSource xs, const GemvLaunch& a);
// Row stride of a PARTIALS output and number of groups of a k-wide input.
size_t gemv_partial_stride(int n);
int gemv_groups(int k);
// y = (base ? base : 0) + ((0 + P[0]) + P[1] + ...), elementwise.
lq8_status launch_combine(hipStream_t s, const float* base, const float* partials, int groups, size_t stride, int n,
                          float* y);

// Grouped GEMV over independent problems (device-side descriptor table).
struct GemvProblemDev {
    const int8_t* codes;
    const uint16_t* scales;
    const float* x;
    float* y;
    int n, k, tile_begin, pad;
};
lq8_status launch_gemv_grouped(hipStream_t s, const GemvProblemDev* d_probs, int count, int total_tiles,
                               int max_k);

// Activation quantization into the tiled layout (codes + f32 scales).
lq8_status launch_quantize_act(hipStream_t s, const float* x, int m, int k, int8_t* codes, float* scales32);
// AoS quantization (public device quantizer).
lq8_status launch_quantize_aos(hipStream_t s, const float* x, size_t nblocks, uint8_t* blocks);
// W8A8 GEMM: y[m, n] (+ resid) from tiled activations and a tiled weight.
lq8_status launch_gemm(hipStream_t s, const int8_t* xq, const float* xs, int m, const lq8_weight* w, float* y,
                       const float* resid, int ldy, int col0);

lq8_status launch_repack_aos(hipStream_t s, const uint8_t* aos, size_t n_rows, size_t nb, size_t row0,
                             const lq8_weight* w);
lq8_status launch_unpack_aos(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint8_t* aos);
lq8_status launch_quantize_weight_f32(hipStream_t s, const float* src, size_t n_rows, size_t row0,
                                      const lq8_weight* w);
lq8_status launch_random_weight(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint64_t seed,
                                uint64_t stream, float stddev);
lq8_status launch_dequant_rows(hipStream_t s, const lq8_weight* w, const uint32_t* d_ids, size_t row0,
                               size_t nrows, float* y);


// ---- decoder support kernels (model_kernels.hip) ---------------------------
// positions: pos_i = (d_pos ? *d_pos : pos_base) + i
struct QkRopeLaunch {
    const float* qkv;      // [n][q_dim + 2*kv_dim] projections (q | k | v)
    const float* q_norm;   // [head_dim]
    const float* k_norm;   // [head_dim]
    const float* cos_t;    // [max_pos][head_dim/2]
    const float* sin_t;
    float* q_out;          // [n][q_dim] normalized, rotated queries
    float* k_cache;        // [kv_heads][max_pos][head_dim] (this layer)
    float* v_cache;        // [kv_heads][max_pos][head_dim] (this layer)
    const int* d_pos;
    int pos_base, n, num_heads, num_kv_heads, head_dim, max_pos;
    float eps;
};
lq8_status launch_qk_rope_kv(hipStream_t s, const QkRopeLaunch& a);

struct AttnLaunch {
    const float* q;        // [n][num_heads*head_dim]
    const float* k_cache;
    const float* v_cache;
    float* out;            // [n][num_heads*head_dim]
    const int* d_pos;
    int pos_base, n, num_heads, num_kv_heads, head_dim, max_pos;
    float scale;
};
lq8_status launch_attention(hipStream_t s, const AttnLaunch& a);

// Attention with head_dim 128 and at most 2 q-heads per kv head, one
// workgroup per (kv head, query row).  Decode form: qkv_p holds the qkv
// projection as qkv_g partials of stride qkv_stride; the kernel normalizes
// and rotates q/k, appends k/v at the position and attends.  Prefill form:
// q_rows holds normalized, rotated queries and the cache is filled.
struct AttnGroupLaunch {
    const float* qkv_p;
    int qkv_g;
    size_t qkv_stride;
    const float* q_rows;
    const float* q_norm;
    const float* k_norm;
    const float* cos_t;
    const float* sin_t;
    float* k_cache;        // [kv_heads][max_pos][128] (this layer)
    float* v_cache;
    float* out;            // [n][num_heads * 128]
    const int* d_pos;
    int pos_base, n, num_heads, num_kv_heads, max_pos;
    float eps, scale;
};
lq8_status launch_attention_group(hipStream_t s, const AttnGroupLaunch& a);
bool attention_group_supported(int num_heads, int num_kv_heads, int head_dim, int max_pos);

lq8_status launch_rms_norm_rows(hipStream_t s, const float* x, const float* w, int rows, int dim, float eps, float* y);
lq8_status launch_silu_mul(hipStream_t s, const float* gu, int rows, int inter, float* act);
lq8_status launch_silu(hipStream_t s, const float* x, size_t n, float* y);
// Argmax with last-index ties over logits[n]; writes tokens_out[*d_step] and
// *d_tok, then advances *d_pos and *d_step (all device scalars).
lq8_status launch_argmax_step(hipStream_t s, const float* logits, int n, uint32_t* d_tok, uint32_t* tokens_out,
                              int* d_pos, int* d_step);

// ---- allocation helpers ----------------------------------------------------
lq8_status weight_alloc(lq8_ctx* ctx, size_t n_out, size_t k_in, lq8_weight** out);
void weight_release(lq8_weight* w);

}  // namespace lq8
