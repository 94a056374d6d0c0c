// lq8_internal.h -- shared definitions of the gfx950 Q8_0 library.
//
// Device layout of a Q8_0 weight W[n_out, k_in] (nb = k_in / 32 blocks per
// row, np = ceil(nb / 2) block pairs; rows grouped into 16-row tiles):
//   codes  [tiles][np][part 0..3][16 rows][16 int8]      1 KiB per (tile, pair)
//          part = (block & 1) * 2 + half: codes 16*half .. 16*half + 15 of
//          block 2*pair + (part >> 1)
//   scales [tiles][2 * np][16 rows] f16 bits
// Lane l of a wave reading one (tile, pair) chunk with a 16-byte load gets
// row l % 16, part l / 16: one 1 KiB coalesced load covers 16 rows x 2
// blocks.  The same chunk is the A/B operand layout of the int8 MFMA GEMM
// (rows 0..15 and 16..31 of a 32-row MFMA tile come from two tiles).
// Padding rows (n_out .. 16 * tiles) and the padding block of an odd nb are
// zero codes with a zero scale.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/lq8.h"

namespace lq8 {

constexpr int QK = 32;
constexpr int BLOCK_BYTES = 34;
constexpr int TILE_ROWS = 16;
constexpr int CHUNK_BYTES = 1024;   // one (tile, pair) chunk of codes
constexpr int GEMM_GROUP = 8;       // blocks per accumulation group of the W8A8 GEMM
constexpr int GEMV_MAX_K = 12288;  // staged input + group sums stay under 64 KiB of LDS
constexpr int GEMV_LONG_MAX_K = 131072;  // plain inputs above GEMV_MAX_K stream through LDS in stages

__host__ __device__ inline size_t code_off(size_t tile, size_t np, size_t b, int half, int r) {
    return ((tile * np + (b >> 1)) * 64 + ((b & 1) * 2 + half) * 16 + r) * 16;
}
__host__ __device__ inline size_t scale_off(size_t tile, size_t np, size_t b, int r) {
    return (tile * 2 * np + b) * 16 + r;
}

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
    // host-pointer linear forward: device and pinned host staging of x and y,
    // grown on demand (never per call)
    void* io_dev = nullptr;
    void* io_host = nullptr;
    void* io_host_dev = nullptr;  // io_host as the device addresses it (mapped pinned memory)
    size_t io_bytes = 0;
};

struct lq8_weight {
    lq8_ctx* ctx = nullptr;
    size_t n_out = 0, k_in = 0, nb = 0, np = 0, tiles = 0;
    int8_t* codes = nullptr;
    uint16_t* scales = nullptr;
};

namespace lq8 {

// Scratch owned by the context; grows on demand (synchronizes before growing).
lq8_status ctx_scratch(lq8_ctx* ctx, size_t bytes, void** out);

// ---- GEMV (gemv.hip) ---------------------------------------------------------
// Input x of a GEMV: plain f32 vector, RmsNorm of a hidden vector,
// silu(gate) * up of a concatenated [gate | up] vector, or the attention
// output combined from per-segment partials (x = partials, see AttnSegLaunch).
enum XSource : int {
    XS_PLAIN = 0, XS_RMSNORM = 1, XS_SILU = 2, XS_ATTN = 3,
    // RMSNorm of x + the pairwise tree over nparts chunk sums (the input of
    // a GEMV whose producer wrote chunk sums, EPI_PART); workgroup 0 stores
    // the joined vector to h_out
    XS_RMSNORM_JOIN = 4,
    // silu(gate) * up over one input chunk (EPI_PART): gate at x, up at x + xk
    XS_SILU_PART = 5
};
// Output: y = W x, y = resid + W x, or y = W x plus the per-tile argmax
// (value, index; last index on ties) of the logits.
// EPI_SWIGLU (multi-vector GEMV only): rows = [gate | up] halves; the
// workgroup of gate tile i also runs up tile i and stores silu(gate) * up
// (rows / 2 outputs per vector).
enum Epilogue : int {
    EPI_STORE = 0, EPI_RESID = 1, EPI_ARGMAX = 2, EPI_SWIGLU = 3,
    // input chunks of part_pairs block pairs (a power of two; workgroup
    // column blockIdx.y = chunk): y[chunk * n + row] receives the chunk sums
    EPI_PART = 4
};

struct GemvArgs {
    const int8_t* codes;
    const uint16_t* scales;
    const float* x;        // XS_PLAIN: x[k]; XS_RMSNORM: hidden[k]; XS_SILU: gu[2k]
    const float* norm_w;   // XS_RMSNORM weight [k]
    float* y;              // [n]
    const float* resid;    // EPI_RESID: [n]
    float* arg_val;        // EPI_ARGMAX: [tiles]
    int* arg_idx;          // EPI_ARGMAX: [tiles]
    int n, k;
    float eps;
    // XS_ATTN: position (device scalar or base), heads, partial rows per segment capacity
    const int* d_pos = nullptr;
    int pos_base = 0, attn_heads = 0, attn_cmax = 0;
    // EPI_PART: pairs per input chunk (the launch has ceil(pairs / part_pairs) chunks)
    int part_pairs = 0;
    // XS_RMSNORM_JOIN: parts[nparts][k] chunk sums added to x by the pairwise
    // tree; h_out[k] receives x + that sum
    const float* parts = nullptr;
    int nparts = 0;
    float* h_out = nullptr;
    // set by the kernel for a chunk: pairs per weight row, the chunk's first
    // pair, the offset of up from gate (XS_SILU_PART)
    int npw = 0, p0 = 0, xk = 0;
};
lq8_status launch_gemv(hipStream_t s, XSource xs, Epilogue epi, const GemvArgs& a);

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
// Multi-vector GEMV: each workgroup owns one 16-row tile of one problem and
// applies it to that problem's vectors, each in the single-vector GEMV order
// (so every output equals launch_gemv on that vector).  Problems are the
// routed experts of a MoE layer (lists written on the device) or one dense
// weight applied to a batch of vectors.
struct MvArgs {
    const int8_t* codes;    // problem e's tiles start at tile e * prob_tiles
    const uint16_t* scales;
    int rows, k;            // output rows per problem, input length
    int prob_tiles;
    const int* n_prob;      // device: problem count (null: 1)
    const int* prob_id;     // device: weight index of problem j (null: j)
    const int* vec_begin;   // device: first slots entry of problem j (null: 0)
    const int* vec_count;   // device: vectors of problem j (null: nvec)
    const int* slots;       // device: slot ids (null: slot = entry index)
    int nvec;
    const float* x;         // vector of slot s: x + (s / x_div) * x_stride
    int x_stride, x_div;
    float* y;               // output of slot s: y + s * y_stride
    int y_stride;
    const float* resid;     // EPI_RESID: y = resid[s] + acc, resid + s * resid_stride
    int resid_stride;
    const float* norm_w;    // XS_RMSNORM
    float eps;
    int max_vec = 0;        // upper bound of vectors per problem (1: single-vector pipelined variant)
};
// max_probs: grid rows of problems (n_prob on the device may be smaller);
// vsplit: workgroups per tile sharing the vectors of a problem.
lq8_status launch_gemv_mv(hipStream_t s, XSource xs, Epilogue epi, const MvArgs& a, int max_probs, int vsplit);

// Batch-1 routed expert down projections fused with their combine:
// out[row] = h2[row] + sum over the K experts in ascending index of
// rw[rank] * (down_expert(rank) x[rank])[row].
constexpr int MOE_DOWN_MAX_K = 16;
struct MoeDownArgs {
    const int8_t* codes;    // expert e's tiles start at tile e * prob_tiles
    const uint16_t* scales;
    int rows, k;            // hidden size, expert intermediate size
    int prob_tiles;
    const uint32_t* rids;   // device [K]: expert of each rank
    const float* rw;        // device [K]: routing weight of each rank
    int K;
    const float* x;         // rank q's input: x + q * x_stride
    int x_stride;
    const float* h2;        // residual [rows]
    float* out;             // [rows]
};
bool moe_down_combine_supported(int K, int k);
lq8_status launch_moe_down_combine(hipStream_t s, const MoeDownArgs& a);

// Batch-1 routed expert gate and up projections with the RMSNorm fused:
// y[q][row] = silu(gate_e(n)[row]) * up_e(n)[row], e = rids[q],
// n = RmsNorm(x) -- the values launch_gemv_mv gives (XS_RMSNORM, EPI_SWIGLU)
// for one token.  The weight interleaves gate and up by 8 rows per tile.
struct MoeGateUpArgs {
    const int8_t* codes;    // expert e's tiles start at tile e * prob_tiles (gate, up interleaved by 8)
    const uint16_t* scales;
    int inter, k;           // expert intermediate size (gate rows), hidden size
    int prob_tiles;         // 2 * inter / 16
    const uint32_t* rids;   // device [K]: expert of each rank
    int K;
    const float* x;         // the token's hidden state [k]
    const float* norm_w;    // [k]
    float eps;
    float* y;               // rank q's output: y + q * y_stride (y_stride >= inter)
    int y_stride;
};
bool moe_gate_up1_supported(int K, int inter, int k);
lq8_status launch_moe_gate_up1(hipStream_t s, const MoeGateUpArgs& a);

// Final greedy pick over the per-tile argmax partials: token -> *d_tok and
// tokens_out[*d_step], then *d_pos and *d_step advance (device scalars).
lq8_status launch_argmax_final(hipStream_t s, const float* arg_val, const int* arg_idx, int count, uint32_t* d_tok,
                               uint32_t* tokens_out, int* d_pos, int* d_step);

// ---- Q8_0 format, activation quantization, GEMM (q8_kernels.hip) -------------
// Activation rows x[m, k] -> tiled codes (as a weight, 2 * ceil(m/32) tiles) + f16
// scales in the GEMM's operand layout (act_scale_bytes).
lq8_status launch_quantize_act(hipStream_t s, const float* x, int m, int k, int8_t* codes, uint32_t* scales);
// The same operand from RmsNorm(x) rows (the values launch_rms_norm_rows gives)
// and from silu(gate) * up of [gate | up] rows (the values launch_silu_mul gives).
bool rms_quantize_supported(int dim);
lq8_status launch_rms_quantize_act(hipStream_t s, const float* x, const float* w, int m, int dim, float eps,
                                   int8_t* codes, uint32_t* scales);
lq8_status launch_silu_quantize_act(hipStream_t s, const float* gu, int m, int inter, int8_t* codes,
                                    uint32_t* scales);
// Routed expert outputs y (rows t * K + j) combined into out = h2 + sum of
// w * y (ascending expert index, the values k_moe_combine gives), then the
// operand launch_rms_quantize_act gives for out with norm weight w.
bool combine_rms_quant_supported(int K, int dim);
lq8_status launch_combine_rms_quant(hipStream_t s, const float* h2, const float* eo, const uint32_t* rids,
                                    const float* rw, int K, int m, int dim, const float* w, float eps, float* out,
                                    int8_t* codes, uint32_t* scales);
// The attention outputs of launch_attention_combine (head_dim 128) quantized
// straight into the operand layout: the values launch_attention_combine
// followed by launch_quantize_act give.
lq8_status launch_attention_combine_quant(hipStream_t s, const float* part, size_t part_stride, const int* d_pos,
                                          int batch, int num_heads, int cmax, int8_t* codes, uint32_t* scales);
size_t act_code_bytes(int m, int k);
size_t act_scale_bytes(int m, int k);
// The activation operand back to GGUF blocks [m][k / 32] (tests, inspection).
lq8_status launch_unpack_act(hipStream_t s, const int8_t* codes, const uint32_t* scales, int m, int k,
                             uint8_t* blocks);
// AoS quantization (public device quantizer).
lq8_status launch_quantize_aos(hipStream_t s, const float* x, size_t nblocks, uint8_t* blocks);
// W8A8 GEMM: y[m, n] (+ resid) from tiled activations and a tiled weight.
lq8_status launch_gemm(hipStream_t s, const int8_t* xq, const uint32_t* xs, int m, const lq8_weight* w, float* y,
                       const float* resid);

// ---- sampling (sample.hip) -----------------------------------------------------
struct SampleCfg {
    float temperature;  // 0: greedy
    int top_k;          // 0: all
    float top_p;        // >= 1: off
    float penalty;      // repetition penalty (1: off)
    unsigned long long seed;
};
struct SampleLaunch {
    const float* logits;
    int vocab;
    const uint32_t* counts;   // occurrences of each token so far (penalty; null: none)
    uint32_t* counts_out;     // incremented at the chosen token (null: not kept)
    const SampleCfg* cfg;     // device
    int* d_step;              // device: the RNG counter and output index (advances)
    uint32_t* d_tok;          // device: the token
    uint32_t* tokens_out;     // device [steps] (null: not kept)
    int* d_pos;               // device position, advanced (null: none)
    void* work;               // device, sample_work_bytes(vocab): sort buffers, histograms, chunk sums
    bool topk;                // host: sample_topk_path(config) -- candidate selection instead of the full sort
};
// GenerationConfig ranges (src/generate.rs:96-128) -> the device config.
lq8_status check_sampling(const lq8_sampling* c, SampleCfg* out);
// T > 0 and 1 <= top_k <= 1024: the top-k candidates are selected and sorted
// alone (same rule, same result as the full sort)
bool sample_topk_path(const SampleCfg& c);
size_t sample_work_bytes(int vocab);
// bytes at the start of the workspace that must be zero before its first use
// (the top-k path's histogram and counter; every top-k pick clears them again)
size_t sample_work_zero_bytes(int vocab);
bool sample_vocab_ok(size_t vocab);  // 1 .. 2^20
lq8_status launch_sample(hipStream_t s, const SampleLaunch& a);

// A tensor's rows in a weight: row r at row0 + r, or, with run > 0, in runs of
// `run` rows every `stride` rows (row0 + (r / run) * stride + r % run).
struct RowRun {
    size_t run = 0, stride = 0;
};
__host__ __device__ inline size_t map_row(size_t row0, size_t r, RowRun m) {
    return m.run ? row0 + (r / m.run) * m.stride + r % m.run : row0 + r;
}
lq8_status launch_repack_aos(hipStream_t s, const uint8_t* aos, size_t n_rows, size_t row0, const lq8_weight* w,
                             RowRun rr = {});
lq8_status launch_unpack_aos(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint8_t* aos,
                             RowRun rr = {});
lq8_status launch_quantize_weight_f32(hipStream_t s, const float* src, size_t n_rows, size_t row0,
                                      const lq8_weight* w);
lq8_status launch_quantize_weight_bf16(hipStream_t s, const uint16_t* src, size_t n_rows, size_t row0,
                                       const lq8_weight* w);
lq8_status launch_random_weight(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint64_t seed,
                                uint64_t stream, float stddev, RowRun rr = {});
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

// Attention (head_dim 128, G = num_heads / num_kv_heads <= ATT_MAX_GROUP
// query heads per kv head), positions in segments of ATT_SEG.
// threadIdx.x as a value the compiler must treat as produced here: index
// math derived from it stays next to its use instead of being hoisted out of
// enclosing loops (in a persistent kernel: held in registers through every
// phase).
__device__ __forceinline__ int tid_here() {
    int x = (int)threadIdx.x;
    asm volatile("" : "+v"(x));
    return x;
}

// Workgroup barrier that orders LDS only: the wave waits for its own LDS and
// scalar memory operations (lgkmcnt) and meets the others at s_barrier, but
// not for its global stores (a __syncthreads() also waits for those, a whole
// memory round trip for write-through stores).  The asm's memory clobber
// keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

constexpr int ATT_SEG = 64;
constexpr int ATT_THREADS = 512;
constexpr int ATT_F4 = ATT_SEG * 32 / ATT_THREADS;  // float4 of one segment's K (or V) per thread
constexpr int ATT_PART_STRIDE = 132;                // o_c[128], m_c, l_c, pad
constexpr int ATT_MAX_GROUP = 16;
constexpr int ATT_EARLY_SEGS = 4;                  // decode: segments whose K/V loads precede the position
bool attention_supported(int num_heads, int num_kv_heads, int head_dim);

// Decode: one workgroup per (kv head, segment); normalizes and rotates q/k
// from the qkv projection, appends k/v at the position, and writes per
// (segment, q head) partials part[(c * num_heads + h) * ATT_PART_STRIDE]
// that the o-projection GEMV combines (XS_ATTN).
struct AttnSegLaunch {
    const float* qkv;      // [q_dim + 2 * kv_dim]
    const float* q_norm;
    const float* k_norm;
    const float* cos_t;    // [max_pos][64]
    const float* sin_t;
    float* k_cache;        // [kv_heads][max_pos][128] (this layer)
    float* v_cache;
    float* part;           // [ceil(max_pos / ATT_SEG)][num_heads][ATT_PART_STRIDE]
    const int* d_pos;      // [batch] (null: every sequence at pos_base)
    int pos_base, num_heads, num_kv_heads, max_pos;
    float eps, scale;
    // independent sequences (grid z): sequence b reads qkv + b * qkv_stride,
    // owns k/v_cache + b * kv_stride and writes part + b * part_stride
    int batch = 1;
    size_t qkv_stride = 0, kv_stride = 0, part_stride = 0;
    // query heads per workgroup (0: the num_heads / num_kv_heads of a kv head;
    // a divisor of it spreads one kv head's heads over several workgroups)
    int head_group = 0;
};
lq8_status launch_attention_seg(hipStream_t s, const AttnSegLaunch& a);
// Attention outputs from the per-segment partials of launch_attention_seg,
// for each sequence: out[b][h * 128 + d], combined in segment order with the
// running update of the o-projection's XS_ATTN staging.
lq8_status launch_attention_combine(hipStream_t s, const float* part, size_t part_stride, const int* d_pos,
                                    int batch, int num_heads, int cmax, float* out);

// Prefill: one workgroup per (kv head, query row) over a filled cache.
struct AttnRowsLaunch {
    const float* q_rows;   // [n][num_heads * 128] normalized, rotated
    const float* k_cache;
    const float* v_cache;
    float* out;            // [n][num_heads * 128]
    int pos_base, n, num_heads, num_kv_heads, max_pos;
    float scale;
};
lq8_status launch_attention_rows(hipStream_t s, const AttnRowsLaunch& a);

lq8_status launch_rms_norm_rows(hipStream_t s, const float* x, const float* w, int rows, int dim, float eps, float* y);
lq8_status launch_silu_mul(hipStream_t s, const float* gu, int rows, int inter, float* act);
lq8_status launch_silu(hipStream_t s, const float* x, size_t n, float* y);

// ---- allocation helpers ----------------------------------------------------
lq8_status weight_alloc(lq8_ctx* ctx, size_t n_out, size_t k_in, lq8_weight** out);
void weight_release(lq8_weight* w);

}  // namespace lq8
