/*
 * lq8_oracle.h -- CPU oracle for the Q8_0 hot path (TEST INFRASTRUCTURE).
 *
 * This library is the parity checker.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it.  The shipped library
 * (liblq8.so) never links, loads or calls it.
 *
 * Every float operation below is written out in a fixed order so that the
 * HIP kernels, which follow the same orders, reproduce the results bit for
 * bit.  The orders are documented per function in lq8_oracle.c.
 */
#ifndef LQ8_ORACLE_H
#define LQ8_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK 32          /* elements per Q8_0 block */
#define ORC_BLOCK_BYTES 34 /* f16 scale + 32 int8 codes (GGUF block_q8_0) */
#define ORC_GROUP_BLOCKS 8 /* blocks per accumulation group */

/* ---- scalar numerics ---- */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
float orc_bf16_round(float x);
float orc_expf(float x);
void orc_f32_to_f16_n(const float* x, uint16_t* h, size_t n);
void orc_f16_to_f32_n(const uint16_t* h, float* x, size_t n);
void orc_bf16_round_n(const float* x, float* y, size_t n);
void orc_expf_n(const float* x, float* y, size_t n);

/* 0 = canonical orders (what the GPU computes), 1 = the reference's plain
 * sequential sums.  Global switch, used only to compare the two. */
void orc_set_sequential_sums(int on);
/* 1: the decoder's softmax and SiLU use the C library's expf (the
 * reference's f32::exp on linux-gnu); 0 (default): orc_expf. */
void orc_set_libm_exp(int on);
/* 1 (default) = RmsNorm's bf16 roundings as the reference; 0 = skipped (tests
 * that pin the decoder structure against a float64 restatement). */
void orc_set_bf16_rounding(int on);
/* 1 (default) = rows > 1 through the W8A8 GEMM; 0 = every row through the
 * W8A32 GEMV (the same structure-pinning tests). */
void orc_set_activation_quantization(int on);
void orc_set_threads(int n);

/* ---- Q8_0 format ---- */
int orc_quantize_q8_0(const float* x, size_t n, uint8_t* blocks);
int orc_dequantize_q8_0(const uint8_t* blocks, size_t n, float* y);

/* ---- Q8_0 matmul, W[n_out, k_in] in AoS blocks ---- */
int orc_gemv_q8_0(const uint8_t* w, size_t n_out, size_t k_in, const float* x, float* y);
int orc_gemm_q8_0(const uint8_t* w, size_t n_out, size_t k_in, const float* x, size_t m, float* y);
int orc_linear_forward(const uint8_t* w, size_t n_out, size_t k_in, const float* x, size_t m, float* y);

/* ---- support ops ---- */
int orc_rms_norm(const float* x, const float* weight, size_t rows, size_t dim, float eps, float* y);
int orc_rope_tables(size_t head_dim, size_t max_pos, double theta, float* cos_t, float* sin_t);
int orc_rope_apply(const float* x, size_t heads, size_t seq, size_t head_dim, const float* cos_t,
                   const float* sin_t, size_t offset, float* y);
float orc_silu(float x);
uint32_t orc_argmax_last(const float* x, size_t n);
/* the library's sampling rule (see lq8_sample_device); -1 on bad input */
int64_t orc_sample(const float* logits, size_t V, const uint32_t* counts, float T, uint32_t top_k, float top_p,
                   float penalty, uint64_t seed, uint32_t step);

/* ---- Qwen3 model ---- */
typedef struct {
    uint32_t vocab_size, hidden_size, intermediate_size, num_layers;
    uint32_t num_heads, num_kv_heads, head_dim, max_positions;
    float rms_norm_eps;
    double rope_theta;
} orc_qwen3_config;

/* Tensor table order (pointers are copied, not the data):
 *   [0] embed_tokens Q8_0 [vocab, hidden] (tied lm_head)
 *   [1] final norm f32 [hidden]
 *   per layer l, base = 2 + 11*l:
 *   +0 input_layernorm f32 [hidden]   +1 post_attention_layernorm f32 [hidden]
 *   +2 q_norm f32 [head_dim]           +3 k_norm f32 [head_dim]
 *   +4 q_proj Q8_0  +5 k_proj  +6 v_proj  +7 o_proj
 *   +8 gate_proj    +9 up_proj +10 down_proj                               */
typedef struct orc_model orc_model;
orc_model* orc_model_new(const orc_qwen3_config* cfg, const void* const* tensors);
void orc_model_free(orc_model* m);
void orc_model_clear_kv_cache(orc_model* m);
int orc_model_forward(orc_model* m, const uint32_t* ids, size_t n, size_t offset, float* logits);
int orc_model_forward_with_intermediates(orc_model* m, const uint32_t* ids, size_t n, size_t offset, float* hidden,
                                         float* final_norm, float* logits);
int orc_generate_greedy(orc_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                        uint32_t* out_tokens, float* out_margins);
/* feed_first = 1: the reference's loop as written (every decode step
 * forwards the first generated token, src/generate.rs:632-650). */
int orc_generate_greedy_ex(orc_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new, int feed_first,
                           uint32_t* out_tokens, float* out_margins);

/* ---- Qwen3-MoE decoder layers (decode step of T independent sequences) ----
 * Tensor table, per layer l, base = (8 + 3 * num_experts) * l:
 *   +0 input_layernorm f32 [hidden]  +1 post_attention_layernorm f32 [hidden]
 *   +2 q_norm f32 [head_dim]          +3 k_norm f32 [head_dim]
 *   +4 q_proj  +5 k_proj  +6 v_proj  +7 o_proj  (Q8_0)
 *   +8 + e gate_proj of expert e, +8 + E + e up_proj, +8 + 2E + e down_proj
 * Sequence t of a batch owns KV cache slot t; it is written at pos[t]. */
typedef struct {
    uint32_t hidden_size, num_heads, num_kv_heads, head_dim;
    uint32_t num_experts, top_k, expert_intermediate_size, max_positions, max_batch, num_layers;
    float rms_norm_eps;
    double rope_theta;
} orc_moe_config;
typedef struct orc_moe orc_moe;
orc_moe* orc_moe_new(const orc_moe_config* cfg, const void* const* tensors);
void orc_moe_free(orc_moe* m);
int orc_moe_route(const float* scores, size_t T, size_t E, size_t k, uint32_t* ids, float* weights);
int orc_moe_forward(orc_moe* m, float* hidden, const float* scores, const uint32_t* pos, size_t T);

#ifdef __cplusplus
}
#endif
#endif
