/*
 * lq8.h -- C ABI of the MI355X (gfx950) Q8_0 quantized-weight path.
 *
 * Drop-in boundary for lluda-inference's linear layers.  Each entry point
 * names the reference interface it replaces (paths relative to the
 * reference crate root, lluda-inference/).  Plain pointers and sizes only.
 *
 * Conventions
 *   - Every function returns lq8_status; on failure lq8_last_error() holds a
 *     message for the calling thread.  There is never a silent CPU fallback
 *     (GPU_DESIGN_PRINCIPLES.md:5-45): no device -> LQ8_ERR_NO_DEVICE.
 *   - Q8_0 host blocks are GGUF block_q8_0: 2-byte little-endian f16 scale d
 *     followed by 32 int8 codes (34 bytes per 32 values).  Value = d * q.
 *   - A weight W is [n_out, k_in] row-major, as Linear stores it
 *     (src/attention.rs:30-35); linear forward computes y = x W^T.
 *   - *_device functions take device pointers and enqueue on the context's
 *     stream without synchronizing; the others take host pointers and block.
 *   - One context = one HIP stream.  Calls on one context must not overlap
 *     from several threads; distinct contexts are independent.  Weight
 *     handles are immutable after upload.
 */
#ifndef LQ8_H
#define LQ8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors LludaError kinds (src/error.rs:17-97). */
typedef enum {
    LQ8_OK = 0,
    LQ8_ERR_SHAPE_MISMATCH = 1,   /* LludaError::ShapeMismatch */
    LQ8_ERR_DTYPE_MISMATCH = 2,   /* LludaError::DTypeMismatch */
    LQ8_ERR_DIM_OUT_OF_RANGE = 3, /* LludaError::DimOutOfRange */
    LQ8_ERR_INVALID_ARG = 4,      /* LludaError::Msg (bad argument, null, stale handle) */
    LQ8_ERR_NO_DEVICE = 5,        /* GPU init failure (src/gpu/mod.rs:167-174 panics; here an error) */
    LQ8_ERR_DEVICE = 6,           /* HIP runtime error */
    LQ8_ERR_OUT_OF_MEMORY = 7,
    LQ8_ERR_MODEL = 8             /* LludaError::Model */
} lq8_status;

/* Element type of a host tensor handed to a loader. */
typedef enum {
    LQ8_DTYPE_Q8_0 = 0, /* GGUF block_q8_0 rows (34 bytes per 32 values) */
    LQ8_DTYPE_F32 = 1,
    LQ8_DTYPE_BF16 = 2  /* little-endian bf16, as safetensors stores it */
} lq8_dtype;

typedef struct lq8_ctx lq8_ctx;
typedef struct lq8_weight lq8_weight;
typedef struct lq8_model lq8_model;

#define LQ8_QK 32
#define LQ8_BLOCK_BYTES 34

/* ---- library / errors ------------------------------------------------- */
const char* lq8_version(void);
/* Thread-local message of the last failure (src/error.rs Display). */
const char* lq8_last_error(void);
lq8_status lq8_device_count(int* count);

/* ---- host Q8_0 format (no device needed) -------------------------------
 * Replaces: the planned GGUF Q8_0 quantizer
 * (docs/architecture/arch-2026-01-31-qwen3-omni-q8-rust.md:36-39,275-279). */
size_t lq8_q8_0_bytes(size_t n);
lq8_status lq8_quantize_q8_0(const float* x, size_t n, void* blocks_out);
lq8_status lq8_dequantize_q8_0(const void* blocks, size_t n, float* y);

/* ---- context -----------------------------------------------------------
 * Replaces: gpu::get_context / init (src/gpu/mod.rs:129-178). */
lq8_status lq8_init(int device, lq8_ctx** out);
lq8_status lq8_shutdown(lq8_ctx* ctx);
lq8_status lq8_synchronize(lq8_ctx* ctx);
lq8_status lq8_device_alloc(lq8_ctx* ctx, size_t bytes, void** dptr);
lq8_status lq8_device_free(lq8_ctx* ctx, void* dptr);
lq8_status lq8_copy_to_device(lq8_ctx* ctx, void* dst, const void* src, size_t bytes);
lq8_status lq8_copy_to_host(lq8_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Device-to-device copy enqueued on the context stream (no synchronization).
 * No reference counterpart: used as the known-size copy that calibrates HBM
 * traffic counters, and for device-side staging. */
lq8_status lq8_copy_device(lq8_ctx* ctx, void* dst, const void* src, size_t bytes);
/* HIP-event timer on the context stream (the reference's PROFILE timings,
 * src/tensor.rs:824-885, measured on the device instead of wall clock). */
lq8_status lq8_timer_start(lq8_ctx* ctx);
lq8_status lq8_timer_stop(lq8_ctx* ctx, float* elapsed_ms);

/* ---- weights -----------------------------------------------------------
 * Replaces: Linear::new (src/attention.rs:63-71) taking ownership of a
 * weight Tensor; here the weight is uploaded once and repacked into the
 * device layout (the reference re-uploads per call, src/gpu/gemv.rs:347-411). */
lq8_status lq8_weight_upload(lq8_ctx* ctx, const void* blocks, size_t n_out, size_t k_in, lq8_weight** out);
/* Quantizes f32 [n_out, k_in] on the device (bit-exact with lq8_quantize_q8_0). */
lq8_status lq8_weight_quantize_upload(lq8_ctx* ctx, const float* w, size_t n_out, size_t k_in, lq8_weight** out);
/* The same from bf16 rows (checkpoint weights, ModelWeights::from_safetensors,
 * src/loader.rs:68-188): a bf16 value widens exactly to f32, then the Q8_0
 * quantizer runs on the device. */
lq8_status lq8_weight_quantize_upload_bf16(lq8_ctx* ctx, const uint16_t* w, size_t n_out, size_t k_in,
                                           lq8_weight** out);
/* Device N(0, std) weights from a counter-based generator, quantized on the device. */
lq8_status lq8_weight_random(lq8_ctx* ctx, size_t n_out, size_t k_in, uint64_t seed, uint64_t stream, float std,
                             lq8_weight** out);
lq8_status lq8_weight_download(lq8_ctx* ctx, const lq8_weight* w, void* blocks_out);
lq8_status lq8_weight_shape(const lq8_weight* w, size_t* n_out, size_t* k_in);
lq8_status lq8_weight_free(lq8_weight* w);

/* ---- device quantize / dequantize ---------------------------------------
 * Activation quantizer of the W8A8 path, as a standalone op: d_x f32 [n] ->
 * d_blocks AoS Q8_0 on the device.  Bit-exact with lq8_quantize_q8_0. */
lq8_status lq8_quantize_q8_0_device(lq8_ctx* ctx, const float* d_x, size_t n, void* d_blocks);
/* The activation operand of the W8A8 GEMM, as GGUF blocks [m][k / 32]:
 * rows quantized by the very kernels lq8_linear_forward (m > 1) and the
 * model's prefill run, each bit-exact with lq8_quantize_q8_0 of its input.
 *   LQ8_ACT_PLAIN:    rows d_x [m][k] as they are;
 *   LQ8_ACT_RMSNORM:  RmsNorm (src/rms_norm.rs:143-176) of rows d_x [m][k]
 *                     with weight d_w [k] and eps, fused into the quantizer
 *                     (the prefill input norms);
 *   LQ8_ACT_SILU_MUL: silu(gate) * up of rows d_x [m][2k] = [gate | up]
 *                     (src/mlp.rs:151-164), fused (the prefill down input).
 * Works in the context's scratch buffer; enqueued without synchronizing.
 * Replaces: the planned activation quantizer of the Q8_0 matmul
 * (docs/architecture/arch-2026-01-31-qwen3-omni-q8-rust.md:36-39). */
#define LQ8_ACT_PLAIN 0
#define LQ8_ACT_RMSNORM 1
#define LQ8_ACT_SILU_MUL 2
lq8_status lq8_quantize_activations_device(lq8_ctx* ctx, int source, const float* d_x, const float* d_w, size_t m,
                                          size_t k, float eps, void* d_blocks);
/* Rows [row0, row0+nrows) of W dequantized to f32 [nrows, k_in]: the
 * Embedding::forward row gather on a Q8_0 table (src/embedding.rs:137-152). */
lq8_status lq8_weight_dequantize_rows_device(lq8_ctx* ctx, const lq8_weight* w, size_t row0, size_t nrows,
                                             float* d_y);

/* ---- decoder ops (device pointers) -----------------------------------------
 * RmsNorm::forward (src/rms_norm.rs:123-177): rows of dim values, input and
 * output rounded to bf16 (returned as f32 values), weight rounded to bf16. */
lq8_status lq8_rms_norm_device(lq8_ctx* ctx, const float* d_x, const float* d_w, size_t rows, size_t dim, float eps,
                               float* d_y);
/* Tensor::silu, f32 branch (src/tensor.rs:1955-1990): x / (1 + exp(-x)). */
lq8_status lq8_silu_device(lq8_ctx* ctx, const float* d_x, size_t n, float* d_y);

/* ---- linear forward ------------------------------------------------------
 * Replaces: Linear::forward (src/attention.rs:101-136) and the 2-D
 * Tensor::matmul it calls (src/tensor.rs:804-817, 898-981, 2716-2753;
 * GPU: src/gpu/gemv.rs:294, src/gpu/gemm.rs:295).  y[m, n_out] = x[m, k_in] W^T,
 * f32 in and out.  m == 1: W8A32 GEMV.  m > 1: activations quantized to
 * Q8_0 per row, W8A8 int8 MFMA GEMM, int32 per block, f32 rescale. */
lq8_status lq8_linear_forward(lq8_ctx* ctx, const lq8_weight* w, const float* x, size_t m, float* y);
lq8_status lq8_linear_forward_device(lq8_ctx* ctx, const lq8_weight* w, const float* d_x, size_t m, float* d_y);
/* lq8_linear_forward_device that allocates nothing.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * m > 1 activation operand goes to an 8 MiB array of the library's own,
 * one per GPU (held until the process ends): act codes + scales of about
 * 1.25 * m * k_in bytes (e.g. m = 2048 at k_in = 3072), LQ8_ERR_SHAPE_MISMATCH
 * above.  Every call on a GPU shares that array, so calls that overlap on one
 * GPU (two contexts, two threads) race.  Results are bit-identical to
 * lq8_linear_forward_device. */
lq8_status lq8_linear_forward_device_noalloc(lq8_ctx* ctx, const lq8_weight* w, const float* d_x, size_t m,
                                             float* d_y);
/* The two kernels behind it, callable directly (any m for the GEMM). */
lq8_status lq8_gemv_q8_0_device(lq8_ctx* ctx, const lq8_weight* w, const float* d_x, float* d_y);
lq8_status lq8_gemm_q8_0_device(lq8_ctx* ctx, const lq8_weight* w, const float* d_x, size_t m, float* d_y);

/* Independent GEMVs in one launch (routed MoE experts; a batch of linear
 * layers).  No reference counterpart: the reference runs one matmul per call. */
typedef struct {
    const lq8_weight* w;
    const float* x; /* device, k_in floats */
    float* y;       /* device, n_out floats */
} lq8_gemv_problem;
lq8_status lq8_gemv_grouped_device(lq8_ctx* ctx, const lq8_gemv_problem* problems, size_t count);

/* Benchmark harness (examples/benchmark_gemv.rs:13-99 measured on the device):
 * runs `reps` passes over the problems on the context stream and returns the
 * device time in ms.  mode 0: one launch per problem; 1: one grouped launch
 * per pass; 2: mode 0 replayed from a HIP graph; 3: per-launch HIP-event
 * pairs, returning the sum of the launches' own intervals. */
lq8_status lq8_bench_gemv(lq8_ctx* ctx, const lq8_gemv_problem* problems, size_t count, int mode, int reps,
                          float* ms);

/* Microbenchmark of the workgroup-to-workgroup hand-off a persistent decode
 * kernel needs (no reference counterpart): `rounds` rounds of a data
 * exchange between all nwg workgroups of one cooperative launch, each round
 * two grid-wide synchronisations.  kind 0: one counter with agent-scope
 * release/acquire fences; 1: one counter, the data itself written and read
 * with agent-scope atomics (no cache-wide fences); 2: per-XCD counters
 * under a global one; 3: per-XCD counters and per-XCD release flags.
 * Returns the device time per synchronisation, the values read wrong (must
 * be 0) and whether a bounded wait gave up (must be 0). */
lq8_status lq8_bench_grid_sync(lq8_ctx* ctx, int kind, int nwg, int rounds, float* us_per_sync,
                               uint32_t* mismatches, uint32_t* gave_up);

/* Hardware floors the latency-bound kernels are measured against (a
 * diagnostic without counterpart in the reference), on the context stream:
 *   LQ8_FLOOR_EMPTY   reps back-to-back launches of an empty kernel of nwg
 *                     workgroups: *value = us per launch;
 *   LQ8_FLOOR_STREAM  reps read-only passes over `bytes` of device memory by
 *                     nwg workgroups of 512 threads (8 nontemporal 16-byte
 *                     loads in flight per thread): *value = GB/s;
 *   LQ8_FLOOR_CHASE   one thread following min(reps, bytes / 128) links of a
 *                     random cycle through `bytes` (one word per 128-byte
 *                     line): *value = ns per dependent load;
 *   LQ8_FLOOR_STREAM_CHUNKS  as LQ8_FLOOR_STREAM, each workgroup reading one
 *                     contiguous range: *value = GB/s;
 *   LQ8_FLOOR_EMPTY_GRAPH  reps (<= 10000) launches of an empty kernel of nwg
 *                     workgroups captured as one HIP graph and replayed:
 *                     *value = us per graph node.
 * bytes: for the streams and the chase a multiple of 4096, at most 8 GiB
 * (allocated for the call); for the empty kernels the workgroup size in
 * threads (a multiple of 64 up to 1024; 0: 64). */
#define LQ8_FLOOR_EMPTY 0
#define LQ8_FLOOR_STREAM 1
#define LQ8_FLOOR_CHASE 2
#define LQ8_FLOOR_STREAM_CHUNKS 3
#define LQ8_FLOOR_EMPTY_GRAPH 4
lq8_status lq8_bench_floors(lq8_ctx* ctx, int kind, int nwg, size_t bytes, int reps, double* value);

/* Phase timeline of the persistent greedy decode (the default greedy path, see
 * lq8_generate_greedy), a diagnostic without counterpart in the reference:
 * in a library built with LQ8_PERSIST_TRACE (make trace -> liblq8_trace.so)
 * thread 0 of every workgroup stamps the 100 MHz real-time clock at the
 * LQ8_PT_* marks of the fourth step of each launch, for the first
 * LQ8_PTRACE_LAYERS layers (the lm_head marks in layer 0's row); words of
 * marks not passed stay as they were.  out[(wg * LQ8_PTRACE_LAYERS + layer)
 * * LQ8_PTRACE_POINTS + mark], count = LQ8_PTRACE_WG * LQ8_PTRACE_LAYERS *
 * LQ8_PTRACE_POINTS.  Other builds return LQ8_ERR_INVALID_ARG. */
#define LQ8_PTRACE_WG 512
#define LQ8_PTRACE_LAYERS 64
#define LQ8_PTRACE_POINTS 25
enum {
    LQ8_PT_P1_START = 0,     /* RmsNorm + q|k|v: workgroup enters */
    LQ8_PT_P1_NORMED = 1,    /* the layer input has arrived and is normalised */
    LQ8_PT_P2_START = 2,     /* attention: workgroup enters (its q|k|v tile is out) */
    LQ8_PT_P2_QKV_IN = 3,    /* the segment item's q, k, v have arrived */
    LQ8_PT_P2_SCORES = 4,    /* scores and softmax partials done */
    LQ8_PT_P2_PARTIALS = 5,  /* the segment's partials are out */
    LQ8_PT_P3_START = 6,     /* o GEMV: workgroup enters */
    LQ8_PT_P3_STAGED = 7,    /* the attention output has arrived */
    LQ8_PT_P4_START = 8,     /* RmsNorm + gate|up: workgroup enters */
    LQ8_PT_P4_STAGED = 9,    /* h2 has arrived */
    LQ8_PT_P5_START = 10,    /* down GEMV: workgroup enters */
    LQ8_PT_P5_STAGED = 11,   /* silu(gate) * up has arrived */
    LQ8_PT_P5_DONE = 12,     /* the down tile + residual is out */
    LQ8_PT_P6_START = 13,    /* lm_head: workgroup enters */
    LQ8_PT_P6_NORMED = 14,   /* the last layer's output has arrived and is normalised */
    LQ8_PT_P6_DONE = 15,     /* the workgroup's greedy pick is out */
    LQ8_PT_P2_COMBINED = 16, /* attention: the kv head's segments are combined and out (the combining item) */
    LQ8_PT_P2_COMB_FETCHED = 17, /* combine: the other segments' first (m_c, l_c) and o_c words have arrived */
    LQ8_PT_P2_COMB_COEF = 18,    /* combine: the first batch's coefficients are done */
    LQ8_PT_P1_GATHERED = 19,     /* the layer input's words have arrived (before the join and the norm) */
    LQ8_PT_P1_DOT = 20,          /* the q|k|v tile's group sums are in LDS */
    LQ8_PT_P2_ROPED = 21,        /* attention: q and k normalised and rotated */
    LQ8_PT_P3_COMBINED = 22,     /* o item: its heads' segments combined (P3's own combine) */
    LQ8_PT_P4_NORMED = 23,       /* h2 joined and normalised */
    LQ8_PT_P4_DOT = 24           /* the gate|up tiles' group sums are in LDS */
};
lq8_status lq8_persist_trace(lq8_ctx* ctx, uint64_t* out, size_t count);

/* ---- Qwen3 model ---------------------------------------------------------
 * Replaces: Qwen3ForCausalLM::load/forward/clear_kv_cache
 * (src/model.rs:273-302, 345-372, 396-398) and generate() with greedy
 * sampling (src/generate.rs:611-664, 153-174). */
typedef struct {
    uint32_t vocab_size, hidden_size, intermediate_size, num_layers;
    uint32_t num_heads, num_kv_heads, head_dim, max_positions; /* max_positions <= 1048576 */
    float rms_norm_eps;
    double rope_theta;
} lq8_qwen3_config;

/* Tensor table (host pointers), the same order everywhere:
 *   [0] model.embed_tokens.weight   Q8_0 [vocab, hidden] (tied lm_head)
 *   [1] model.norm.weight           f32  [hidden]
 *   layer l, base 2 + 11*l:
 *   +0 input_layernorm f32 [hidden]   +1 post_attention_layernorm f32 [hidden]
 *   +2 self_attn.q_norm f32 [head_dim] +3 self_attn.k_norm f32 [head_dim]
 *   +4 q_proj +5 k_proj +6 v_proj +7 o_proj +8 gate_proj +9 up_proj +10 down_proj (Q8_0)
 * (weight names: src/model.rs:439-538). */
size_t lq8_model_tensor_count(const lq8_qwen3_config* cfg);
lq8_status lq8_model_tensor_bytes(const lq8_qwen3_config* cfg, size_t index, size_t* bytes);
lq8_status lq8_model_create(lq8_ctx* ctx, const lq8_qwen3_config* cfg, const void* const* tensors,
                            lq8_model** out);
/* The same table with a type per tensor (quantize-on-load): matrices may be
 * LQ8_DTYPE_Q8_0 blocks (a GGUF file), or BF16 / F32 rows (a safetensors
 * checkpoint) quantized on the device; norms may be F32 or BF16. */
lq8_status lq8_model_create_typed(lq8_ctx* ctx, const lq8_qwen3_config* cfg, const void* const* tensors,
                                  const int32_t* dtypes, lq8_model** out);
/* Random init as HF does: Linear/Embedding N(0, std) from a seeded counter
 * generator (quantized on the device), RMSNorm weights 1. */
lq8_status lq8_model_create_random(lq8_ctx* ctx, const lq8_qwen3_config* cfg, uint64_t seed, float std,
                                   lq8_model** out);
lq8_status lq8_model_export_tensor(lq8_model* m, size_t index, void* host_out);
lq8_status lq8_model_clear_kv_cache(lq8_model* m);
/* logits: host f32 [vocab] for the last position (or NULL). offset must equal
 * the number of cached positions (prefill_len + generated - 1 in generate()). */
lq8_status lq8_model_forward(lq8_model* m, const uint32_t* ids, size_t n, size_t offset, float* logits);
/* Qwen3Model::forward_with_intermediates (src/model.rs:201-231) plus the
 * logits: hidden [num_layers + 1][n][hidden] (embedding output, then each
 * layer's output), final_norm [n][hidden], logits [vocab] (or NULL). */
lq8_status lq8_model_forward_with_intermediates(lq8_model* m, const uint32_t* ids, size_t n, size_t offset,
                                                float* hidden, float* final_norm, float* logits);

typedef struct {
    double prefill_ms;      /* prompt forward + first token, device time */
    double decode_ms;       /* the max_new-1 single-token steps, device time */
    double decode_tokens_per_s;
    uint32_t used_graph;    /* 1 if the decode step ran as a replayed HIP graph */
    uint32_t used_persistent; /* 1 if the decode steps ran as one persistent kernel (greedy) */
} lq8_gen_stats;
/* Greedy generation; the token loop stays on the device.  out_tokens: max_new.
 * The decode steps run as one persistent cooperative kernel (all steps, all
 * layers, the lm_head and the pick in one launch) when the model's shape
 * fits it: head_dim 128, hidden_size a multiple of 32 up to 2048 (one
 * kernel instance up to 1024, another above), intermediate_size a multiple
 * of 32 whose down-projection split fits (up to 8192 at hidden 2048 on 256
 * workgroups, Qwen3-1.7B's 6144 included), num_heads * 128 <= 2048,
 * num_heads / num_kv_heads <= 16, and a device with cooperative launch;
 * max_positions is not limited.  lq8_persist_plan tells in advance.  By
 * default the kernel runs up to hidden_size 1024 (above, the per-step
 * kernels are faster); the environment variable LQ8_PERSIST=1 runs it
 * wherever the shape fits, LQ8_PERSIST=0 never.  Otherwise one kernel
 * sequence per step runs, replayed as a HIP graph (lq8_gen_stats tells which
 * ran).  Both give the same tokens, bit for bit the same logits.
 * Each decode step forwards the token generated last.  The reference's loop
 * as written does not: the `let next_token` in its loop body
 * (src/generate.rs:650) shadows the binding of src/generate.rs:632 only for
 * the rest of that iteration, so src/generate.rs:647 forwards the FIRST
 * generated token at every step.  lq8_generate_ex with
 * LQ8_GEN_FEED_FIRST_TOKEN reproduces that loop; the two agree only while
 * the model repeats its first token. */
lq8_status lq8_generate_greedy(lq8_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                               uint32_t* out_tokens, lq8_gen_stats* stats);

/* Whether lq8_generate_greedy of a model with this configuration runs as
 * the persistent kernel on num_workgroups workgroups (the library launches
 * one per compute unit), and the kernel's plan for it: the o and down
 * projections' input chunks and its LDS map (in floats).  Host-only: needs
 * no device.  A diagnostic without counterpart in the reference. */
typedef struct {
    uint32_t supported;          /* 1: the persistent kernel runs this shape */
    uint32_t o_chunk_blocks;     /* the o projection's input chunks: blocks each, and how many */
    uint32_t o_chunks;
    uint32_t down_chunk_pairs;   /* the down projection's input chunks: block pairs each, and how many */
    uint32_t down_chunks;
    uint32_t lds_bytes;          /* dynamic LDS per workgroup */
    uint32_t lds_gather_floats;  /* hand-off gathers, from 0 */
    uint32_t lds_xs_offset;      /* the staged GEMV input */
    uint32_t lds_gs_offset;      /* the waves' group sums */
    uint32_t lds_red_offset;     /* reduction words (16) */
    uint32_t lds_attention_floats; /* an attention item's region, from 0 */
    uint32_t lds_combine_floats;   /* the separate segment combine's region, inside the attention item's */
    uint32_t direct_segments;      /* steps with at most this many 64-position segments combine them in the
                                      o projection's items; longer contexts in one combining item per kv head */
} lq8_persist_info;
lq8_status lq8_persist_plan(const lq8_qwen3_config* cfg, uint32_t num_workgroups, lq8_persist_info* out);
/* The per-workgroup greedy picks of the last persistent decode step (back 0)
 * or of the step before it (back 1) of the model's last lq8_generate_greedy
 * call: workgroup w's largest logit over its lm_head rows (the rows of the
 * 16-row tiles t with (t / 8) % P == w, P workgroups; the last index on
 * ties) as f32 bits and its token index.  *count receives P; capacity must
 * be at least P.  A diagnostic without counterpart in the reference (it lets
 * a test compare the kernel's logits at the picked rows with another
 * implementation's). */
lq8_status lq8_model_persist_picks(lq8_model* m, uint32_t back, float* values, uint32_t* indices, size_t capacity,
                                   size_t* count);

/* ---- sampling ----------------------------------------------------------------
 * The fields of GenerationConfig (src/generate.rs:40-128) besides
 * max_new_tokens, plus the RNG seed; GenerationConfig::new's ranges are
 * enforced (temperature >= 0, top_p in [0, 1], repetition_penalty >= 1;
 * LQ8_ERR_INVALID_ARG otherwise).
 * The reference's samplers are argmax stubs (src/generate.rs:191-329); this
 * library samples for real, by this rule:
 *   x = logits with the repetition penalty applied once per earlier
 *       occurrence of each token (src/generate.rs:353-380; off at 1.0);
 *   temperature 0: greedy, the largest x, the last index on ties;
 *   otherwise z = x / temperature; tokens ordered by z descending (ties: the
 *   lower index first); the first top_k kept (all for 0); integer weights
 *   w = floor(2^32 * exp(z - z_max)) (0 for NaN) and prefix sums C of w in
 *   that order, exact in 64 bits; with top_p < 1 the nucleus ends at the
 *   first C >= ceil(C_last * floor(top_p * 2^24) / 2^24) (the whole kept set
 *   for top_p = 1); u24 = SplitMix64(seed + step * 0x9E3779B97F4A7C15) >> 40,
 *   where step is the index of the generated token (0 for the token after
 *   the prompt), r = floor(C_end * u24 / 2^24); the token is the first one
 *   with C > r (the first one when C_end = 0).
 * Unlike the reference's dispatch (src/generate.rs:670-693), temperature 1
 * with no top-k / top-p samples (the stub returns the argmax there). */
typedef struct {
    float temperature;
    uint32_t top_k;
    float top_p;
    float repetition_penalty;
    uint64_t seed;
} lq8_sampling;

/* sample_with_config (src/generate.rs:670-693) on device logits [vocab]:
 * the token goes to *d_token (device).  vocab: 1 .. 2^20.  d_counts: device
 * [vocab] counts of each token generated so far (the repetition penalty;
 * NULL for none); step: the RNG counter.  Works in the context's scratch
 * buffer; blocks until the token is written. */
lq8_status lq8_sample_device(lq8_ctx* ctx, const float* d_logits, size_t vocab, const uint32_t* d_counts,
                             const lq8_sampling* cfg, uint32_t step, uint32_t* d_token);

/* generate (src/generate.rs:611-664) with a sampling configuration: prefill,
 * the first token from the prefill logits, then up to max_new - 1 decode
 * steps, each sampled on the device (the repetition penalty counts the
 * generated tokens, as the reference's generated_tokens).  eos_ids[n_eos]
 * (may be empty): generation ends at the first generated token in the set,
 * which is kept (is_eos_token, src/generate.rs:639-659); *n_out receives the
 * number of tokens written to out_tokens (capacity max_new), and the KV cache
 * is left as the reference's early stop leaves it (the last token is not
 * forwarded).  The loop runs on the device without per-token host
 * synchronisation, so steps after an EOS are computed and discarded. */
lq8_status lq8_generate(lq8_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                        const lq8_sampling* cfg, const uint32_t* eos_ids, size_t n_eos, uint32_t* out_tokens,
                        size_t* n_out, lq8_gen_stats* stats);
/* lq8_generate with flags.  LQ8_GEN_FEED_FIRST_TOKEN: every decode step
 * forwards the first generated token, the reference's generate() loop as
 * written (src/generate.rs:632-650; see lq8_generate_greedy).  Replaces the
 * same generate() as lq8_generate. */
#define LQ8_GEN_FEED_FIRST_TOKEN 1u
lq8_status lq8_generate_ex(lq8_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                           const lq8_sampling* cfg, const uint32_t* eos_ids, size_t n_eos, uint32_t flags,
                           uint32_t* out_tokens, size_t* n_out, lq8_gen_stats* stats);
lq8_status lq8_model_free(lq8_model* m);

/* ---- Qwen3-MoE decoder layers (Qwen3-30B-A3B style), decode steps --------
 * No reference counterpart: the reference has no MoE code.  The layer is
 * assembled from the reference's decoder numerics (src/transformer.rs:180-204,
 * src/attention.rs:318-403, src/mlp.rs:151-164) with a routed expert MLP.
 * A forward call decodes one token for each of T independent sequences
 * (sequence t owns KV cache slot t and writes position pos[t]).  The
 * attention projections follow Linear::forward on the [T, hidden] input: at
 * T = 1 the W8A32 GEMV, at T > 1 the W8A8 GEMM (each row's activations
 * quantized to Q8_0 on their own).  The routed experts run the per-token
 * W8A32 GEMV order at every T.  A token's result therefore depends on
 * whether it runs alone or in a batch (the activation quantization, about
 * 1e-2 relative), never on the other tokens of its batch.
 * Router, from given scores s [T][num_experts] per layer: p = softmax(s)
 * (max, exp(s - max), SUM64 denominator, divide); top_k by p descending,
 * ties to the lower expert index; weights renormalised over the top_k in
 * rank order.  Experts combine in ascending expert index:
 * out = h2 + ((0 + w_a * y_a) + w_b * y_b) + ...  */
typedef struct lq8_moe lq8_moe;
typedef struct {
    uint32_t hidden_size, num_heads, num_kv_heads, head_dim;
    uint32_t num_experts, top_k, expert_intermediate_size;
    uint32_t max_positions; /* KV capacity per sequence, 1 .. 1048576 */
    uint32_t max_batch;     /* sequences per forward call */
    uint32_t num_layers;
    float rms_norm_eps;
    double rope_theta;
} lq8_moe_config;

/* Tensor table (host pointers), layer l at base (8 + 3 * num_experts) * l:
 *   +0 input_layernorm f32 [hidden]  +1 post_attention_layernorm f32 [hidden]
 *   +2 q_norm f32 [head_dim]          +3 k_norm f32 [head_dim]
 *   +4 q_proj +5 k_proj +6 v_proj +7 o_proj (Q8_0)
 *   +8 + e  expert e gate_proj Q8_0 [expert_intermediate, hidden]
 *   +8 + E + e  up_proj (same shape), +8 + 2E + e  down_proj [hidden, expert_intermediate] */
size_t lq8_moe_tensor_count(const lq8_moe_config* cfg);
lq8_status lq8_moe_tensor_bytes(const lq8_moe_config* cfg, size_t index, size_t* bytes);
lq8_status lq8_moe_create(lq8_ctx* ctx, const lq8_moe_config* cfg, const void* const* tensors, lq8_moe** out);
/* Q8_0 weights N(0, std) from a seeded counter generator, norms 1. */
lq8_status lq8_moe_create_random(lq8_ctx* ctx, const lq8_moe_config* cfg, uint64_t seed, float std, lq8_moe** out);
lq8_status lq8_moe_export_tensor(lq8_moe* m, size_t index, void* host_out);
/* Q8_0 bytes of all layers' weights (attention + every expert). */
lq8_status lq8_moe_weight_bytes(lq8_moe* m, size_t* bytes);
/* Device pointers: hidden [T][hidden] (input, overwritten by the last layer's
 * output), scores [num_layers][T][num_experts], pos [T] (each < max_positions).
 * Enqueued on the context stream; no host synchronisation. */
lq8_status lq8_moe_forward_device(lq8_moe* m, float* d_hidden, const float* d_scores, const int32_t* d_pos, size_t T);
/* Host arrays; synchronous. */
lq8_status lq8_moe_forward(lq8_moe* m, float* hidden, const float* scores, const int32_t* pos, size_t T);
/* Routing of the last forward: experts [num_layers][T][top_k] in rank order and
 * their renormalised weights (host arrays). */
lq8_status lq8_moe_routing(lq8_moe* m, uint32_t* experts, float* weights);
/* Zero every KV cache slot. */
lq8_status lq8_moe_clear_kv_cache(lq8_moe* m);
lq8_status lq8_moe_free(lq8_moe* m);

#ifdef __cplusplus
}
#endif
#endif /* LQ8_H */
