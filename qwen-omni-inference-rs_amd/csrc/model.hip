// model.hip -- Qwen3ForCausalLM on Q8_0 weights (src/model.rs, src/transformer.rs,
// src/attention.rs, src/mlp.rs, src/generate.rs of the reference crate).
//
// Weights live once in HBM in the tiled Q8_0 layout.  q/k/v and gate/up are
// stored as one concatenated weight each (rows are independent, so the
// results are those of the separate projections).  Decode (one position)
// runs 5 kernels per layer, each output final when its kernel ends:
//   RmsNorm + qkv GEMV
//   attention per (kv head, 64-position segment): q/k RmsNorm, RoPE, KV append
//   o GEMV on the combined segment partials, + residual
//   RmsNorm + gate|up GEMV
//   silu(gate) * up staged into the down GEMV, + residual
// then RmsNorm + lm_head GEMV with per-tile argmax and one argmax kernel.
// Prefill (n > 1 positions) runs the MFMA GEMM on quantized activations; the
// RmsNorms and silu(gate) * up are fused into the activation quantizer.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <utility>
#include <vector>

#include "decode_persistent.h"
#include "lq8_internal.h"

using namespace lq8;

namespace {

struct Layer {
    lq8_weight *qkv = nullptr, *o = nullptr, *gu = nullptr, *down = nullptr;
    float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

}  // namespace

struct lq8_model {
    lq8_ctx* ctx = nullptr;
    lq8_qwen3_config c{};
    size_t QD = 0, KD = 0, QKV = 0;
    int cmax = 0;  // attention segments at max_positions
    lq8_weight* embed = nullptr;
    float* final_norm = nullptr;
    std::vector<Layer> layers;
    float *cos_t = nullptr, *sin_t = nullptr;
    float *kc = nullptr, *vc = nullptr;  // [layer][kv_head][pos][head_dim] each
    size_t kv_len = 0;
    // single-position buffers
    float *h = nullptr, *h2 = nullptr, *qkv = nullptr, *gu = nullptr, *apart = nullptr, *logits = nullptr;
    // decode's down projection in input chunks of down_cs pairs (down_nch >= 2
    // of them; 0: whole rows): dpart[down_nch][hidden] holds the chunk sums,
    // which the next RMSNorm GEMV joins with the residual
    float* dpart = nullptr;
    int down_cs = 0, down_nch = 0;
    float* arg_val = nullptr;
    int* arg_idx = nullptr;
    uint32_t* d_ids = nullptr;
    size_t ids_cap = 0;
    int *d_pos = nullptr, *d_step = nullptr;
    uint32_t *d_tok = nullptr, *d_tokens = nullptr;
    size_t tokens_cap = 0;
    // prefill buffers, capacity in rows
    size_t pf_cap = 0;
    float *P_h = nullptr, *P_x = nullptr, *P_qkv = nullptr, *P_qr = nullptr, *P_attn = nullptr, *P_gu = nullptr,
          *P_xs = nullptr;
    int8_t* P_xq = nullptr;
    // replayed decode steps, indexed by the token they forward: [0] the token
    // generated last (d_tok), [1] the first generated token (d_tokens[0], the
    // reference loop as written)
    hipGraphExec_t graph[2] = {nullptr, nullptr};
    // sampling: device config, token counts, sort buffers, the sampled decode graphs
    SampleCfg* d_scfg = nullptr;
    uint32_t* d_counts = nullptr;
    uint8_t* s_work = nullptr;  // sampler workspace (sample_work_bytes(vocab))
    hipGraphExec_t sgraph[2] = {nullptr, nullptr};
    bool s_topk = false;            // the sampling path of the next sampler launches (host copy of the choice)
    bool sgraph_topk[2] = {false, false};  // the path each sgraph was captured with
    hipEvent_t e0 = nullptr, e1 = nullptr, e2 = nullptr;
    // persistent greedy decode (decode_persistent.hip): per-layer weight
    // pointers, tagged hand-off buffers, the argument block, the abort flag
    PLayer* d_player = nullptr;
    uint64_t* hand = nullptr;  // qkvb | partb | attb | resb | h2b | actb | argb
    size_t hand_words = 0;
    int last_steps = 0;        // steps of the last persistent launch
    int persist_cdir = 0;      // the plan's direct-combine limit (segments per step)
    PersistArgs* d_pargs = nullptr;  // [2]: the argument blocks of a call's (at most) two launches
    PersistArgs h_pargs{};     // the model's argument block; each launch uploads a copy of it from h_launch
    PersistArgs h_launch[2]{};
    unsigned* d_abort = nullptr;
    unsigned tag = 1;          // tag of the next persistent step (0 never used)
    int persist_wg = 0;        // workgroups of the cooperative launch (0: not set up)
};

namespace {

void drop_graphs(lq8_model* m) {
    for (int i = 0; i < 2; i++) {
        if (m->graph[i]) (void)hipGraphExecDestroy(m->graph[i]);
        if (m->sgraph[i]) (void)hipGraphExecDestroy(m->sgraph[i]);
        m->graph[i] = m->sgraph[i] = nullptr;
    }
}

lq8_status validate(const lq8_qwen3_config* c) {
    if (!c) return fail(LQ8_ERR_INVALID_ARG, "config is null");
    if (!c->vocab_size || !c->hidden_size || !c->intermediate_size || !c->num_layers || !c->num_heads ||
        !c->num_kv_heads || !c->head_dim || !c->max_positions)
        return fail(LQ8_ERR_MODEL, "config: zero dimension");
    if (c->num_heads % c->num_kv_heads) return fail(LQ8_ERR_MODEL, "num_heads must be divisible by num_kv_heads");
    if (c->hidden_size % 32 || c->intermediate_size % 32)
        return fail(LQ8_ERR_MODEL, "hidden and intermediate sizes must be multiples of 32 (Q8_0 blocks)");
    if (!attention_supported((int)c->num_heads, (int)c->num_kv_heads, (int)c->head_dim))
        return fail(LQ8_ERR_MODEL, "attention needs head_dim 128 and at most 16 query heads per kv head");
    // the KV cache holds layers * kv heads * max_positions * 128 floats twice
    // (Qwen3's 40960 positions: 9.4 GB at 0.6B); every position index is 64-bit
    if (c->max_positions > (1u << 20)) return fail(LQ8_ERR_MODEL, "max_positions > 1048576 not supported");
    if (c->hidden_size > (uint32_t)GEMV_MAX_K || c->intermediate_size > (uint32_t)GEMV_MAX_K ||
        c->num_heads * c->head_dim > (uint32_t)GEMV_MAX_K)
        return fail(LQ8_ERR_MODEL, "dimensions above 12288 not supported");
    return LQ8_OK;
}

template <typename T>
lq8_status dalloc(T** p, size_t count) {
    LQ8_HIP(hipMalloc((void**)p, count * sizeof(T) + 16));
    return LQ8_OK;
}

void release(lq8_model* m) {
    if (!m) return;
    registry_remove(m);
    auto F = [](void* p) { if (p) (void)hipFree(p); };
    drop_graphs(m);
    if (m->e0) (void)hipEventDestroy(m->e0);
    if (m->e1) (void)hipEventDestroy(m->e1);
    if (m->e2) (void)hipEventDestroy(m->e2);
    weight_release(m->embed);
    F(m->final_norm);
    for (auto& L : m->layers) {
        weight_release(L.qkv); weight_release(L.o); weight_release(L.gu); weight_release(L.down);
        F(L.in_norm); F(L.post_norm); F(L.q_norm); F(L.k_norm);
    }
    F(m->cos_t); F(m->sin_t); F(m->kc); F(m->vc);
    F(m->h); F(m->h2); F(m->qkv); F(m->gu); F(m->apart); F(m->logits); F(m->arg_val); F(m->arg_idx); F(m->dpart);
    F(m->d_ids); F(m->d_pos); F(m->d_step); F(m->d_tok); F(m->d_tokens);
    F(m->P_h); F(m->P_x); F(m->P_qkv); F(m->P_qr); F(m->P_attn); F(m->P_gu); F(m->P_xs); F(m->P_xq);
    F(m->d_scfg); F(m->d_counts); F(m->s_work);
    F(m->d_player); F(m->hand); F(m->d_pargs); F(m->d_abort);
    delete m;
}

// Allocate weights (uninitialised), norms, tables, caches and decode buffers.
lq8_status build_skeleton(lq8_ctx* ctx, const lq8_qwen3_config* c, lq8_model* m) {
    m->ctx = ctx;
    m->c = *c;
    const size_t Hd = c->hidden_size, I = c->intermediate_size, hd = c->head_dim, P = c->max_positions;
    m->QD = (size_t)c->num_heads * hd;
    m->KD = (size_t)c->num_kv_heads * hd;
    m->QKV = m->QD + 2 * m->KD;
    m->cmax = (int)((P + ATT_SEG - 1) / ATT_SEG);
    lq8_status st;
    if ((st = weight_alloc(ctx, c->vocab_size, Hd, &m->embed))) return st;
    if ((st = dalloc(&m->final_norm, Hd))) return st;
    m->layers.resize(c->num_layers);
    for (auto& L : m->layers) {
        if ((st = weight_alloc(ctx, m->QKV, Hd, &L.qkv))) return st;
        if ((st = weight_alloc(ctx, Hd, m->QD, &L.o))) return st;
        if ((st = weight_alloc(ctx, 2 * I, Hd, &L.gu))) return st;
        if ((st = weight_alloc(ctx, Hd, I, &L.down))) return st;
        if ((st = dalloc(&L.in_norm, Hd)) || (st = dalloc(&L.post_norm, Hd)) || (st = dalloc(&L.q_norm, hd)) ||
            (st = dalloc(&L.k_norm, hd)))
            return st;
    }
    // RoPE tables (src/rope.rs:77-128): f64 math, cast to f32, each frequency twice.
    const size_t R = hd / 2, half = R / 2;
    std::vector<float> ct(P * R), stbl(P * R);
    std::vector<double> inv(half);
    for (size_t i = 0; i < half; i++) inv[i] = 1.0 / std::pow(c->rope_theta, (double)(2 * i) / (double)R);
    for (size_t p = 0; p < P; p++)
        for (size_t i = 0; i < half; i++) {
            const double f = (double)p * inv[i];
            const float cv = (float)std::cos(f), sv = (float)std::sin(f);
            ct[p * R + 2 * i] = ct[p * R + 2 * i + 1] = cv;
            stbl[p * R + 2 * i] = stbl[p * R + 2 * i + 1] = sv;
        }
    if ((st = dalloc(&m->cos_t, P * R)) || (st = dalloc(&m->sin_t, P * R))) return st;
    LQ8_HIP(hipMemcpy(m->cos_t, ct.data(), P * R * sizeof(float), hipMemcpyHostToDevice));
    LQ8_HIP(hipMemcpy(m->sin_t, stbl.data(), P * R * sizeof(float), hipMemcpyHostToDevice));
    const size_t kv = (size_t)c->num_layers * c->num_kv_heads * hd * P;
    if ((st = dalloc(&m->kc, kv)) || (st = dalloc(&m->vc, kv))) return st;
    LQ8_HIP(hipMemset(m->kc, 0, kv * sizeof(float)));
    LQ8_HIP(hipMemset(m->vc, 0, kv * sizeof(float)));
    if ((st = dalloc(&m->h, Hd)) || (st = dalloc(&m->h2, Hd)) || (st = dalloc(&m->qkv, m->QKV)) ||
        (st = dalloc(&m->gu, 2 * I)) || (st = dalloc(&m->apart, (size_t)m->cmax * c->num_heads * ATT_PART_STRIDE)) ||
        (st = dalloc(&m->logits, c->vocab_size)) || (st = dalloc(&m->arg_val, m->embed->tiles)) ||
        (st = dalloc(&m->arg_idx, m->embed->tiles)) || (st = dalloc(&m->d_pos, 1)) || (st = dalloc(&m->d_step, 1)) ||
        (st = dalloc(&m->d_tok, 1)) || (st = dalloc(&m->dpart, 4 * (size_t)Hd)))
        return st;
    {
        // the down projection's 16-row tiles leave compute units idle: input
        // chunks (an aligned power-of-two pair count of at most 128, at most 4
        // chunks) put (tile, chunk) workgroups on them -- the fewest chunks
        // that still give every CU one (each chunk sum is one more vector for
        // the joining GEMV to read): Qwen3-0.6B 3 chunks of 16 pairs, 1.7B 2
        // of 64, 4B 2 of 128
        const int tilesH = Hd / TILE_ROWS, npI = (int)((I / 32 + 1) / 2), ncu = m->ctx->num_cus;
        if (tilesH < ncu && npI > 8) {
            int cs = 8;
            while ((npI + cs - 1) / cs > 4) cs *= 2;
            while (2 * cs <= 128 && 2 * cs < npI && tilesH * ((npI + 2 * cs - 1) / (2 * cs)) >= ncu) cs *= 2;
            if (cs <= 128 && (npI + cs - 1) / cs >= 2) {
                m->down_cs = cs;
                m->down_nch = (npI + cs - 1) / cs;
            }
        }
    }
    LQ8_HIP(hipEventCreate(&m->e0));
    LQ8_HIP(hipEventCreate(&m->e1));
    LQ8_HIP(hipEventCreate(&m->e2));
    return LQ8_OK;
}

lq8_status fill_norm(float* d, size_t n, const float* host) {
    if (host) {
        LQ8_HIP(hipMemcpy(d, host, n * sizeof(float), hipMemcpyHostToDevice));
    } else {
        std::vector<float> ones(n, 1.0f);
        LQ8_HIP(hipMemcpy(d, ones.data(), n * sizeof(float), hipMemcpyHostToDevice));
    }
    return LQ8_OK;
}

// Tensor index -> (weight, first row, rows) or norm buffer.
struct TensorRef {
    lq8_weight* w = nullptr;
    size_t row0 = 0, rows = 0;
    float* norm = nullptr;
    size_t norm_len = 0;
};

TensorRef tensor_ref(lq8_model* m, size_t idx) {
    TensorRef t;
    const size_t Hd = m->c.hidden_size, I = m->c.intermediate_size, hd = m->c.head_dim;
    if (idx == 0) { t.w = m->embed; t.rows = m->c.vocab_size; return t; }
    if (idx == 1) { t.norm = m->final_norm; t.norm_len = Hd; return t; }
    const size_t l = (idx - 2) / 11, k = (idx - 2) % 11;
    Layer& L = m->layers[l];
    switch (k) {
        case 0: t.norm = L.in_norm; t.norm_len = Hd; break;
        case 1: t.norm = L.post_norm; t.norm_len = Hd; break;
        case 2: t.norm = L.q_norm; t.norm_len = hd; break;
        case 3: t.norm = L.k_norm; t.norm_len = hd; break;
        case 4: t.w = L.qkv; t.row0 = 0; t.rows = m->QD; break;
        case 5: t.w = L.qkv; t.row0 = m->QD; t.rows = m->KD; break;
        case 6: t.w = L.qkv; t.row0 = m->QD + m->KD; t.rows = m->KD; break;
        case 7: t.w = L.o; t.rows = Hd; break;
        case 8: t.w = L.gu; t.row0 = 0; t.rows = I; break;
        case 9: t.w = L.gu; t.row0 = I; t.rows = I; break;
        default: t.w = L.down; t.rows = Hd; break;
    }
    return t;
}

lq8_status ensure_ids(lq8_model* m, size_t n) {
    if (n > m->ids_cap) {
        LQ8_HIP(hipStreamSynchronize(m->ctx->stream));
        if (m->d_ids) LQ8_HIP(hipFree(m->d_ids));
        m->d_ids = nullptr;
        lq8_status st = dalloc(&m->d_ids, n);
        if (st) return st;
        m->ids_cap = n;
    }
    return LQ8_OK;
}

lq8_status ensure_prefill(lq8_model* m, size_t n) {
    if (n <= m->pf_cap) return LQ8_OK;
    LQ8_HIP(hipStreamSynchronize(m->ctx->stream));
    auto F = [](float*& p) { if (p) (void)hipFree(p); p = nullptr; };
    F(m->P_h); F(m->P_x); F(m->P_qkv); F(m->P_qr); F(m->P_attn); F(m->P_gu); F(m->P_xs);
    if (m->P_xq) (void)hipFree(m->P_xq);
    m->P_xq = nullptr;
    m->pf_cap = 0;
    const size_t Hd = m->c.hidden_size, I = m->c.intermediate_size;
    const int kmax = (int)std::max(Hd, std::max(m->QD, (size_t)I));
    lq8_status st;
    if ((st = dalloc(&m->P_h, n * Hd)) || (st = dalloc(&m->P_x, n * Hd)) || (st = dalloc(&m->P_qkv, n * m->QKV)) ||
        (st = dalloc(&m->P_qr, n * m->QD)) || (st = dalloc(&m->P_attn, n * m->QD)) ||
        (st = dalloc(&m->P_gu, n * 2 * I)) ||
        (st = dalloc(&m->P_xs, act_scale_bytes((int)n, kmax) / sizeof(float))) ||
        (st = dalloc(&m->P_xq, act_code_bytes((int)n, kmax))))
        return st;
    m->pf_cap = n;
    return LQ8_OK;
}

lq8_status trace_copy(lq8_model* m, float* host, const float* dev, size_t count) {
    if (!host) return LQ8_OK;
    LQ8_HIP(hipMemcpyAsync(host, dev, count * sizeof(float), hipMemcpyDeviceToHost, m->ctx->stream));
    return LQ8_OK;
}

GemvArgs gemv_args(const lq8_weight* w, const float* x, float* y) {
    GemvArgs a{w->codes, w->scales, x, nullptr, y, nullptr, nullptr, nullptr, (int)w->n_out, (int)w->k_in, 0.0f};
    return a;
}

// One position through the decoder (src/model.rs:170-195 with L = 1) and the
// lm_head GEMV with per-tile argmax partials; the token id and the position
// come from device memory (d_pos null: position pos_base).
// trace (optional, host): [0] embedding output, [1 + l] output of layer l.
lq8_status enqueue_decode(lq8_model* m, const uint32_t* d_id, const int* d_pos, int pos_base, float* trace = nullptr,
                          float* final_hidden = nullptr) {
    hipStream_t s = m->ctx->stream;
    const lq8_qwen3_config& c = m->c;
    const int Hd = (int)c.hidden_size;
    const size_t layer_kv = (size_t)c.num_kv_heads * c.head_dim * c.max_positions;
    const float scale = 1.0f / std::sqrt((float)c.head_dim);
    lq8_status st;
    // down in input chunks (not while tracing the layers' outputs, which the
    // chunk sums would only give one launch later); LQ8_DOWN_CHUNKS=0: whole rows
    const char* dce = std::getenv("LQ8_DOWN_CHUNKS");
    const bool chunks = m->down_nch >= 2 && !trace && !(dce && dce[0] == '0');
    if ((st = launch_dequant_rows(s, m->embed, d_id, 0, 1, m->h))) return st;
    if ((st = trace_copy(m, trace, m->h, Hd))) return st;
    for (size_t l = 0; l < m->layers.size(); l++) {
        Layer& L = m->layers[l];
        // input_layernorm + q|k|v projection (src/transformer.rs:190; src/attention.rs:330-332);
        // after a chunked down projection the layer input h = h2 + its chunk
        // sums (joined here, in the GEMV block tree, and stored to h)
        const bool join = chunks && l > 0;
        GemvArgs g1 = gemv_args(L.qkv, join ? m->h2 : m->h, m->qkv);
        g1.norm_w = L.in_norm;
        g1.eps = c.rms_norm_eps;
        if (join) {
            g1.parts = m->dpart;
            g1.nparts = m->down_nch;
            g1.h_out = m->h;
        }
        if ((st = launch_gemv(s, join ? XS_RMSNORM_JOIN : XS_RMSNORM, EPI_STORE, g1))) return st;
        // q/k norm, RoPE, KV append, attention per segment (src/attention.rs:336-399)
        AttnSegLaunch at{m->qkv, L.q_norm, L.k_norm, m->cos_t, m->sin_t, m->kc + l * layer_kv, m->vc + l * layer_kv,
                         m->apart, d_pos, pos_base, (int)c.num_heads, (int)c.num_kv_heads, (int)c.max_positions,
                         c.rms_norm_eps, scale};
        if ((st = launch_attention_seg(s, at))) return st;
        // o_proj on the combined attention output, + residual (src/transformer.rs:194)
        GemvArgs g2 = gemv_args(L.o, m->apart, m->h2);
        g2.resid = m->h;
        g2.d_pos = d_pos;
        g2.pos_base = pos_base;
        g2.attn_heads = (int)c.num_heads;
        g2.attn_cmax = m->cmax;
        if ((st = launch_gemv(s, XS_ATTN, EPI_RESID, g2))) return st;
        // post_attention_layernorm + gate|up (src/transformer.rs:197; src/mlp.rs:153,157)
        GemvArgs g3 = gemv_args(L.gu, m->h2, m->gu);
        g3.norm_w = L.post_norm;
        g3.eps = c.rms_norm_eps;
        if ((st = launch_gemv(s, XS_RMSNORM, EPI_STORE, g3))) return st;
        // down(silu(gate) * up) + residual (src/mlp.rs:163; src/transformer.rs:203):
        // whole rows, or the chunk sums that the next RMSNorm GEMV joins
        if (chunks) {
            GemvArgs g4 = gemv_args(L.down, m->gu, m->dpart);
            g4.part_pairs = m->down_cs;
            if ((st = launch_gemv(s, XS_SILU_PART, EPI_PART, g4))) return st;
        } else {
            GemvArgs g4 = gemv_args(L.down, m->gu, m->h);
            g4.resid = m->h2;
            if ((st = launch_gemv(s, XS_SILU, EPI_RESID, g4))) return st;
        }
        if ((st = trace_copy(m, trace ? trace + (l + 1) * Hd : nullptr, m->h, Hd))) return st;
    }
    if (final_hidden && !chunks)
        LQ8_HIP(hipMemcpyAsync(final_hidden, m->h, Hd * sizeof(float), hipMemcpyDeviceToDevice, s));
    // final norm -> lm_head logits + per-tile argmax (src/model.rs:357-371)
    GemvArgs g5 = gemv_args(m->embed, chunks ? m->h2 : m->h, m->logits);
    g5.norm_w = m->final_norm;
    g5.eps = c.rms_norm_eps;
    g5.arg_val = m->arg_val;
    g5.arg_idx = m->arg_idx;
    if (chunks) {
        g5.parts = m->dpart;
        g5.nparts = m->down_nch;
        g5.h_out = m->h;
    }
    if ((st = launch_gemv(s, chunks ? XS_RMSNORM_JOIN : XS_RMSNORM, EPI_ARGMAX, g5))) return st;
    if (final_hidden && chunks)
        LQ8_HIP(hipMemcpyAsync(final_hidden, m->h, Hd * sizeof(float), hipMemcpyDeviceToDevice, s));
    return LQ8_OK;
}

lq8_status quant_gemm(lq8_model* m, const float* x, int n, const lq8_weight* w, float* y, const float* resid) {
    hipStream_t s = m->ctx->stream;
    uint32_t* xs = reinterpret_cast<uint32_t*>(m->P_xs);
    lq8_status st = launch_quantize_act(s, x, n, (int)w->k_in, m->P_xq, xs);
    if (st) return st;
    return launch_gemm(s, m->P_xq, xs, n, w, y, resid);
}

// GEMM input RmsNorm(h) rows: the norm is fused into the activation quantizer
// (the same operand as rms_norm_rows followed by quantize_act) where the
// hidden size allows it.
lq8_status norm_quant_gemm(lq8_model* m, const float* h, const float* norm_w, int n, const lq8_weight* w, float* y) {
    hipStream_t s = m->ctx->stream;
    const int Hd = (int)m->c.hidden_size;
    if (!rms_quantize_supported(Hd)) {
        lq8_status st = launch_rms_norm_rows(s, h, norm_w, n, Hd, m->c.rms_norm_eps, m->P_x);
        return st ? st : quant_gemm(m, m->P_x, n, w, y, nullptr);
    }
    uint32_t* xs = reinterpret_cast<uint32_t*>(m->P_xs);
    lq8_status st = launch_rms_quantize_act(s, h, norm_w, n, Hd, m->c.rms_norm_eps, m->P_xq, xs);
    return st ? st : launch_gemm(s, m->P_xq, xs, n, w, y, nullptr);
}

// n positions starting at pos_base (src/model.rs:170-195), then the last
// position's logits and per-tile argmax partials.
lq8_status enqueue_prefill(lq8_model* m, int n, int pos_base, float* trace = nullptr) {
    hipStream_t s = m->ctx->stream;
    const lq8_qwen3_config& c = m->c;
    const int Hd = (int)c.hidden_size, I = (int)c.intermediate_size;
    const size_t layer_kv = (size_t)c.num_kv_heads * c.head_dim * c.max_positions;
    const float scale = 1.0f / std::sqrt((float)c.head_dim);
    lq8_status st;
    if ((st = launch_dequant_rows(s, m->embed, m->d_ids, 0, n, m->P_h))) return st;
    if ((st = trace_copy(m, trace, m->P_h, (size_t)n * Hd))) return st;
    for (size_t l = 0; l < m->layers.size(); l++) {
        Layer& L = m->layers[l];
        if ((st = norm_quant_gemm(m, m->P_h, L.in_norm, n, L.qkv, m->P_qkv))) return st;
        QkRopeLaunch qr{m->P_qkv, L.q_norm, L.k_norm, m->cos_t, m->sin_t, m->P_qr, m->kc + l * layer_kv,
                        m->vc + l * layer_kv, nullptr, pos_base, n, (int)c.num_heads, (int)c.num_kv_heads,
                        (int)c.head_dim, (int)c.max_positions, c.rms_norm_eps};
        if ((st = launch_qk_rope_kv(s, qr))) return st;
        AttnRowsLaunch at{m->P_qr, m->kc + l * layer_kv, m->vc + l * layer_kv, m->P_attn, pos_base, n,
                          (int)c.num_heads, (int)c.num_kv_heads, (int)c.max_positions, scale};
        if ((st = launch_attention_rows(s, at))) return st;
        if ((st = quant_gemm(m, m->P_attn, n, L.o, m->P_h, m->P_h))) return st;
        if ((st = norm_quant_gemm(m, m->P_h, L.post_norm, n, L.gu, m->P_gu))) return st;
        if ((st = launch_silu_quantize_act(s, m->P_gu, n, I, m->P_xq, reinterpret_cast<uint32_t*>(m->P_xs))))
            return st;
        if ((st = launch_gemm(s, m->P_xq, reinterpret_cast<const uint32_t*>(m->P_xs), n, L.down, m->P_h, m->P_h)))
            return st;
        if (trace && (st = trace_copy(m, trace + (l + 1) * (size_t)n * Hd, m->P_h, (size_t)n * Hd))) return st;
    }
    // final norm + lm_head on the last position only (src/model.rs:357-371)
    GemvArgs g = gemv_args(m->embed, m->P_h + (size_t)(n - 1) * Hd, m->logits);
    g.norm_w = m->final_norm;
    g.eps = c.rms_norm_eps;
    g.arg_val = m->arg_val;
    g.arg_idx = m->arg_idx;
    return launch_gemv(s, XS_RMSNORM, EPI_ARGMAX, g);
}

lq8_status launch_pick(lq8_model* m) {
    return launch_argmax_final(m->ctx->stream, m->arg_val, m->arg_idx, (int)m->embed->tiles, m->d_tok, m->d_tokens,
                               m->d_pos, m->d_step);
}

// Sampling buffers (allocated on first use, vocabulary-sized).
lq8_status ensure_sampler(lq8_model* m) {
    if (m->d_scfg && m->d_counts && m->s_work) return LQ8_OK;
    // a failed earlier attempt may have left some of them: start over (and
    // drop any graph that captured the old buffers)
    for (auto& g : m->sgraph) {
        if (g) (void)hipGraphExecDestroy(g);
        g = nullptr;
    }
    auto F = [](void* p) { if (p) (void)hipFree(p); };
    F(m->d_scfg); F(m->d_counts); F(m->s_work);
    m->d_scfg = nullptr;
    m->d_counts = nullptr;
    m->s_work = nullptr;
    const int V = (int)m->c.vocab_size;
    lq8_status st;
    if ((st = dalloc(&m->d_scfg, 1)) || (st = dalloc(&m->d_counts, (size_t)V)) ||
        (st = dalloc(&m->s_work, sample_work_bytes(V))))
        return st;
    return LQ8_OK;
}

// sample_with_config on the model's logits: the token -> d_tok and
// d_tokens[*d_step]; d_step, d_pos and the token's count advance.
lq8_status launch_sample_pick(lq8_model* m) {
    SampleLaunch a{};
    a.logits = m->logits;
    a.vocab = (int)m->c.vocab_size;
    a.counts = m->d_counts;
    a.counts_out = m->d_counts;
    a.cfg = m->d_scfg;
    a.d_step = m->d_step;
    a.d_tok = m->d_tok;
    a.tokens_out = m->d_tokens;
    a.d_pos = m->d_pos;
    a.work = m->s_work;
    a.topk = m->s_topk;
    return launch_sample(m->ctx->stream, a);
}

// The decode step's input token: the one generated last, or (feed_first) the
// first generated token, which the reference's loop forwards at every step.
const uint32_t* step_token(lq8_model* m, bool feed_first) { return feed_first ? m->d_tokens : m->d_tok; }

lq8_status capture_sample_graph(lq8_model* m, bool feed_first) {
    hipGraphExec_t& slot = m->sgraph[feed_first];
    if (slot && m->sgraph_topk[feed_first] == m->s_topk) return LQ8_OK;
    if (slot) {
        (void)hipGraphExecDestroy(slot);
        slot = nullptr;
    }
    hipStream_t s = m->ctx->stream;
    hipGraph_t g = nullptr;
    LQ8_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
    lq8_status st = enqueue_decode(m, step_token(m, feed_first), m->d_pos, 0);
    if (!st) st = launch_sample_pick(m);
    hipError_t e = hipStreamEndCapture(s, &g);
    if (st) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&slot, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        slot = nullptr;
        return hip_fail(e, "hipGraphInstantiate");
    }
    m->sgraph_topk[feed_first] = m->s_topk;
    return LQ8_OK;
}

lq8_status capture_decode_graph(lq8_model* m, bool feed_first) {
    hipGraphExec_t& slot = m->graph[feed_first];
    if (slot) return LQ8_OK;
    hipStream_t s = m->ctx->stream;
    hipGraph_t g = nullptr;
    LQ8_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
    lq8_status st = enqueue_decode(m, step_token(m, feed_first), m->d_pos, 0);
    if (!st) st = launch_pick(m);
    hipError_t e = hipStreamEndCapture(s, &g);
    if (st) {
        if (g) (void)hipGraphDestroy(g);
        return st;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    e = hipGraphInstantiate(&slot, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) {
        slot = nullptr;
        return hip_fail(e, "hipGraphInstantiate");
    }
    return LQ8_OK;
}

}  // namespace

namespace {

PersistShape persist_shape(const lq8_model* m) {
    const lq8_qwen3_config& c = m->c;
    return PersistShape{(int)c.hidden_size, (int)c.intermediate_size, (int)c.num_heads, (int)c.num_kv_heads,
                        (int)c.head_dim, (int)c.max_positions};
}

// Workgroups of the persistent launch: one per compute unit, or fewer when
// LQ8_PERSIST_WG names a smaller count (a test of the kernel's other work
// splits).
int persist_target_wg(const lq8_model* m) {
    const int P = m->ctx->num_cus;
    const char* e = std::getenv("LQ8_PERSIST_WG");
    const int want = e != nullptr ? std::atoi(e) : 0;
    return want > 0 && want < P ? want : P;
}

// Whether greedy decode runs as the persistent kernel: by default where the
// shape is supported up to hidden 1024 (its first instance; above, the
// replayed per-step kernels with the down projection in input chunks are
// faster: Qwen3-1.7B shapes 1075 against 1007 tok/s); LQ8_PERSIST=1 wherever
// the shape is supported, LQ8_PERSIST=0 never (the per-step kernels,
// replayed as a graph, or as plain launches under LQ8_NO_GRAPH).
bool persist_wanted(const lq8_model* m) {
    const char* e = std::getenv("LQ8_PERSIST");
    if (e != nullptr && e[0] == '0') return false;
    if (!(e != nullptr && e[0] == '1') && m->c.hidden_size > 1024) return false;
    return persist_supported(persist_shape(m), persist_target_wg(m));
}

// Device state of the persistent decode (allocated once per model and
// workgroup count).
lq8_status persist_setup(lq8_model* m) {
    const int P = persist_target_wg(m);
    if (m->persist_wg == P) return LQ8_OK;
    if (m->persist_wg) {
        // set up for another workgroup count: start again from zeroed words
        LQ8_HIP(hipStreamSynchronize(m->ctx->stream));
        LQ8_HIP(hipFree(m->d_player));
        LQ8_HIP(hipFree(m->hand));
        m->d_player = nullptr;
        m->hand = nullptr;
        m->persist_wg = 0;
        m->tag = 1;
        m->last_steps = 0;
    }
    const lq8_qwen3_config& c = m->c;
    int coop = 0;
    LQ8_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, m->ctx->device));
    if (!coop) return fail(LQ8_ERR_DEVICE, "persistent decode: no cooperative launch on this device");
    const PersistShape sh = persist_shape(m);
    PersistLayout lay{};
    if (!persist_layout(sh, P, &lay)) return fail(LQ8_ERR_MODEL, "persistent decode: shape not supported");
    const size_t L = c.num_layers, H = c.hidden_size, I = c.intermediate_size, NH = c.num_heads;
    const size_t cmax = (size_t)m->cmax;
    const size_t qkv = L * m->QKV, part = L * cmax * NH * ATT_PART_STRIDE, att = L * NH * 128,
                 res = (L + 1) * (1 + lay.nchO) * H, h2 = L * (1 + lay.nchD) * H, act = L * I, arg = 4 * (size_t)P;
    m->hand_words = qkv + part + att + res + h2 + act + arg;
    std::vector<PLayer> pl(L);
    for (size_t l = 0; l < L; l++) {
        const Layer& Ly = m->layers[l];
        pl[l] = PLayer{Ly.qkv->codes, Ly.o->codes, Ly.gu->codes, Ly.down->codes, Ly.qkv->scales, Ly.o->scales,
                       Ly.gu->scales, Ly.down->scales, Ly.in_norm, Ly.post_norm, Ly.q_norm, Ly.k_norm};
    }
    lq8_status st;
    if ((st = dalloc(&m->d_player, L)) || (st = dalloc(&m->hand, m->hand_words)) ||
        (!m->d_pargs && (st = dalloc(&m->d_pargs, 2))) || (!m->d_abort && (st = dalloc(&m->d_abort, 1))))
        return st;
    LQ8_HIP(hipMemcpy(m->d_player, pl.data(), L * sizeof(PLayer), hipMemcpyHostToDevice));
    LQ8_HIP(hipMemset(m->hand, 0, m->hand_words * sizeof(uint64_t)));  // tag 0: never a step's
    PersistArgs& a = m->h_pargs;
    a = PersistArgs{};
    a.layers = m->d_player;
    a.L = (int)L;
    a.emb_c = m->embed->codes;
    a.emb_s = m->embed->scales;
    a.final_norm = m->final_norm;
    a.cos_t = m->cos_t;
    a.sin_t = m->sin_t;
    a.kc = m->kc;
    a.vc = m->vc;
    a.H = (int)H; a.I = (int)I; a.NH = (int)NH; a.NKV = (int)c.num_kv_heads;
    a.max_pos = (int)c.max_positions; a.cmax = m->cmax; a.vocab = (int)c.vocab_size;
    a.eps = c.rms_norm_eps;
    a.scale = 1.0f / std::sqrt((float)c.head_dim);
    a.csO = lay.csO;
    a.nchO = lay.nchO;
    a.csD = lay.csD;
    a.nchD = lay.nchD;
    a.cdir = lay.cdir;
    m->persist_cdir = lay.cdir;
    a.qkvb = m->hand;
    a.partb = a.qkvb + qkv;
    a.attb = a.partb + part;
    a.resb = a.attb + att;
    a.h2b = a.resb + res;
    a.actb = a.h2b + h2;
    a.argb = a.actb + act;
    a.abort_flag = m->d_abort;
    a.fr = lay.fr;
    a.xs_off = lay.xs_off;
    a.gs_off = lay.gs_off;
    a.red_off = lay.red_off;
    a.smem_bytes = lay.smem_bytes;
    m->persist_wg = P;
    return LQ8_OK;
}

// The decode steps of generate() at positions pos0 .. pos0 + steps - 1 (the
// input token is in d_tok; tokens_out[1 + s] gets step s's pick): the steps
// whose positions have at most cdir segments as one cooperative launch of the
// kernel instance without the combining items, the later ones as a launch of
// the instance with them.  The host argument blocks stay unchanged until the
// caller synchronizes the stream.
lq8_status launch_persist(lq8_model* m, int pos0, int steps, bool feed_first) {
    hipStream_t s = m->ctx->stream;
    if ((uint64_t)m->tag + (uint64_t)steps >= 0xFFFFFF00ull) {  // tags wrap: clear every word back to tag 0
        LQ8_HIP(hipMemsetAsync(m->hand, 0, m->hand_words * sizeof(uint64_t), s));
        m->tag = 1;
        m->last_steps = 0;
    }
    // LQ8_PERSIST_CDIR lowers the direct-combine limit (0: every step through
    // the combining attention items), a test of both paths on one shape
    const char* e = std::getenv("LQ8_PERSIST_CDIR");
    const int cdir = e != nullptr ? std::min(std::max(std::atoi(e), 0), m->persist_cdir) : m->persist_cdir;
    // steps at positions below cdir * ATT_SEG have at most cdir segments
    const int n_short = std::max(0, std::min(steps, cdir * ATT_SEG - pos0));
    LQ8_HIP(hipMemsetAsync(m->d_abort, 0, sizeof(unsigned), s));
    const int ch5 = m->h_pargs.csD / (PERSIST_THREADS / 64);
    for (int part = 0; part < 2; part++) {
        const int first = part == 0 ? 0 : n_short, n = part == 0 ? n_short : steps - n_short;
        if (n == 0) continue;
        PersistArgs& a = m->h_launch[part];
        a = m->h_pargs;
        a.cdir = cdir;
        a.pos0 = pos0 + first;
        a.steps = n;
        a.step0 = 1 + first;
        a.feed_first = feed_first ? 1 : 0;
        a.tag0 = m->tag + (unsigned)first;
        a.d_tok = m->d_tok;
        a.tokens_out = m->d_tokens;
        a.d_pos = m->d_pos;
        a.d_step = m->d_step;
        LQ8_HIP(hipMemcpyAsync(m->d_pargs + part, &a, sizeof(PersistArgs), hipMemcpyHostToDevice, s));
        lq8_status st = launch_decode_persistent(s, m->d_pargs + part, a.smem_bytes, m->persist_wg, ch5,
                                                 persist_pairs_per_wave(a.H), part == 1);
        if (st) return st;
    }
    m->tag += (unsigned)steps;
    m->last_steps = steps;
    return LQ8_OK;
}

// generate (src/generate.rs:611-664): greedy picks (sc null) or sampled ones;
// feed_first: every decode step forwards the first generated token.
lq8_status run_generate(lq8_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new, const SampleCfg* sc,
                        bool feed_first, uint32_t* out_tokens, lq8_gen_stats* stats) {
    if (!prompt || n_prompt == 0) return fail(LQ8_ERR_INVALID_ARG, "empty prompt");
    if (max_new == 0 || !out_tokens) return fail(LQ8_ERR_INVALID_ARG, "max_new must be positive");
    if (n_prompt + max_new - 1 > m->c.max_positions)
        return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "prompt + generated tokens exceed max_positions");
    for (size_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= m->c.vocab_size) return fail(LQ8_ERR_INVALID_ARG, "token id out of range for vocab_size");
    LQ8_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    lq8_status st;
    if ((st = ensure_ids(m, n_prompt))) return st;
    if (max_new > m->tokens_cap) {
        if (m->d_tokens) LQ8_HIP(hipFree(m->d_tokens));
        m->d_tokens = nullptr;
        if ((st = dalloc(&m->d_tokens, max_new))) return st;
        m->tokens_cap = max_new;
        drop_graphs(m);  // they captured the old token buffer
    }
    if (n_prompt > 1 && (st = ensure_prefill(m, n_prompt))) return st;
    const bool use_graph = std::getenv("LQ8_NO_GRAPH") == nullptr;
    if (sc && (st = ensure_sampler(m))) return st;
    if (sc) m->s_topk = sample_topk_path(*sc);
    const bool use_persist = !sc && max_new > 1 && persist_wanted(m);
    if (!use_persist) m->last_steps = 0;  // the picks on record are no longer this call's
    if (use_persist && (st = persist_setup(m))) return st;
    if (!use_persist && use_graph && max_new > 1 &&
        (st = sc ? capture_sample_graph(m, feed_first) : capture_decode_graph(m, feed_first)))
        return st;
    // clear_kv_cache (src/generate.rs:618), then prefill at offset 0
    m->kv_len = 0;
    const int zero = 0, pos0 = (int)n_prompt - 1;
    LQ8_HIP(hipMemcpyAsync(m->d_ids, prompt, n_prompt * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    LQ8_HIP(hipMemcpyAsync(m->d_step, &zero, sizeof(int), hipMemcpyHostToDevice, s));
    LQ8_HIP(hipMemcpyAsync(m->d_pos, &pos0, sizeof(int), hipMemcpyHostToDevice, s));
    if (sc) {
        // the penalty counts the generated tokens only (generated_tokens, src/generate.rs:627-660)
        LQ8_HIP(hipMemcpyAsync(m->d_scfg, sc, sizeof(SampleCfg), hipMemcpyHostToDevice, s));
        LQ8_HIP(hipMemsetAsync(m->d_counts, 0, m->c.vocab_size * sizeof(uint32_t), s));
        LQ8_HIP(hipMemsetAsync(m->s_work, 0, sample_work_zero_bytes((int)m->c.vocab_size), s));
    }
    LQ8_HIP(hipEventRecord(m->e0, s));
    st = n_prompt == 1 ? enqueue_decode(m, m->d_ids, nullptr, 0) : enqueue_prefill(m, (int)n_prompt, 0);
    if (st) return st;
    // first token from the prefill logits; d_pos becomes n_prompt
    if ((st = sc ? launch_sample_pick(m) : launch_pick(m))) return st;
    LQ8_HIP(hipEventRecord(m->e1, s));
    if (use_persist && (st = launch_persist(m, (int)n_prompt, (int)max_new - 1, feed_first))) return st;
    for (size_t t = 1; t < max_new && !use_persist; t++) {
        if (use_graph) {
            LQ8_HIP(hipGraphLaunch(sc ? m->sgraph[feed_first] : m->graph[feed_first], s));
        } else {
            if ((st = enqueue_decode(m, step_token(m, feed_first), m->d_pos, 0))) return st;
            if ((st = sc ? launch_sample_pick(m) : launch_pick(m))) return st;
        }
    }
    LQ8_HIP(hipEventRecord(m->e2, s));
    LQ8_HIP(hipMemcpyAsync(out_tokens, m->d_tokens, max_new * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    unsigned aborted = 0;
    if (use_persist) LQ8_HIP(hipMemcpyAsync(&aborted, m->d_abort, sizeof(unsigned), hipMemcpyDeviceToHost, s));
    LQ8_HIP(hipStreamSynchronize(s));
    if (aborted) {
        // the tags an aborted launch leaves are not
        // trusted: the next launch starts from zeroed words
        LQ8_HIP(hipMemsetAsync(m->hand, 0, m->hand_words * sizeof(uint64_t), s));
        LQ8_HIP(hipStreamSynchronize(s));
        m->tag = 1;
        m->last_steps = 0;
        return fail(LQ8_ERR_DEVICE, "persistent decode: a workgroup hand-off did not arrive in time (aborted)");
    }
    m->kv_len = n_prompt + max_new - 1;
    if (stats) {
        float a = 0, b = 0;
        LQ8_HIP(hipEventElapsedTime(&a, m->e0, m->e1));
        LQ8_HIP(hipEventElapsedTime(&b, m->e1, m->e2));
        stats->prefill_ms = a;
        stats->decode_ms = b;
        stats->decode_tokens_per_s = (max_new > 1 && b > 0) ? (double)(max_new - 1) / (b * 1e-3) : 0.0;
        stats->used_graph = (use_graph && !use_persist) ? 1u : 0u;
        stats->used_persistent = use_persist ? 1u : 0u;
    }
    return LQ8_OK;
}

}  // namespace

#define CHECK_M(m) \
    if (!registry_has(m)) return fail(LQ8_ERR_INVALID_ARG, "invalid or released model handle")

extern "C" {

size_t lq8_model_tensor_count(const lq8_qwen3_config* cfg) { return cfg ? 2 + 11 * (size_t)cfg->num_layers : 0; }

lq8_status lq8_model_tensor_bytes(const lq8_qwen3_config* c, size_t idx, size_t* bytes) {
    if (!c || !bytes) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (idx >= lq8_model_tensor_count(c)) return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "tensor index out of range");
    const size_t Hd = c->hidden_size, I = c->intermediate_size, hd = c->head_dim;
    const size_t QD = c->num_heads * hd, KD = c->num_kv_heads * hd;
    auto q8 = [](size_t r, size_t k) { return r * (k / 32) * 34; };
    if (idx == 0) { *bytes = q8(c->vocab_size, Hd); return LQ8_OK; }
    if (idx == 1) { *bytes = Hd * 4; return LQ8_OK; }
    switch ((idx - 2) % 11) {
        case 0: case 1: *bytes = Hd * 4; break;
        case 2: case 3: *bytes = hd * 4; break;
        case 4: *bytes = q8(QD, Hd); break;
        case 5: case 6: *bytes = q8(KD, Hd); break;
        case 7: *bytes = q8(Hd, QD); break;
        case 8: case 9: *bytes = q8(I, Hd); break;
        default: *bytes = q8(Hd, I); break;
    }
    return LQ8_OK;
}

lq8_status lq8_model_create_typed(lq8_ctx* ctx, const lq8_qwen3_config* cfg, const void* const* tensors,
                                  const int32_t* dtypes, lq8_model** out) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid context handle");
    if (!tensors || !out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    lq8_status st = validate(cfg);
    if (st) return st;
    const size_t count = lq8_model_tensor_count(cfg);
    for (size_t i = 0; i < count; i++) {
        if (!tensors[i]) return fail(LQ8_ERR_INVALID_ARG, "null tensor in table");
        if (dtypes && dtypes[i] != LQ8_DTYPE_Q8_0 && dtypes[i] != LQ8_DTYPE_F32 && dtypes[i] != LQ8_DTYPE_BF16)
            return fail(LQ8_ERR_DTYPE_MISMATCH, "unknown tensor dtype");
    }
    LQ8_HIP(hipSetDevice(ctx->device));
    lq8_model* m = new lq8_model();
    registry_add(m);
    if ((st = build_skeleton(ctx, cfg, m))) { release(m); return st; }
    void* tmp = nullptr;
    size_t tmp_cap = 0;
    std::vector<float> widened;
    for (size_t i = 0; i < count && !st; i++) {
        TensorRef t = tensor_ref(m, i);
        const int dt = dtypes ? dtypes[i] : (t.norm ? LQ8_DTYPE_F32 : LQ8_DTYPE_Q8_0);
        if (t.norm) {
            if (dt == LQ8_DTYPE_Q8_0) { st = fail(LQ8_ERR_DTYPE_MISMATCH, "norm weights must be F32 or BF16"); break; }
            const float* host = (const float*)tensors[i];
            if (dt == LQ8_DTYPE_BF16) {  // widen on the host (exact)
                const uint16_t* b = (const uint16_t*)tensors[i];
                widened.resize(t.norm_len);
                for (size_t j = 0; j < t.norm_len; j++) {
                    const uint32_t u = (uint32_t)b[j] << 16;
                    std::memcpy(&widened[j], &u, 4);
                }
                host = widened.data();
            }
            st = fill_norm(t.norm, t.norm_len, host);
            continue;
        }
        const size_t k = t.w->nb * 32;
        const size_t bytes = dt == LQ8_DTYPE_Q8_0 ? t.rows * t.w->nb * BLOCK_BYTES
                             : dt == LQ8_DTYPE_F32 ? t.rows * k * sizeof(float)
                                                   : t.rows * k * sizeof(uint16_t);
        if (bytes > tmp_cap) {
            if (tmp) (void)hipFree(tmp);
            tmp = nullptr;
            hipError_t e = hipMalloc(&tmp, bytes);
            if (e != hipSuccess) { st = hip_fail(e, "staging"); break; }
            tmp_cap = bytes;
        }
        hipError_t e = hipMemcpy(tmp, tensors[i], bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) { st = hip_fail(e, "tensor upload"); break; }
        if (dt == LQ8_DTYPE_Q8_0) st = launch_repack_aos(ctx->stream, (const uint8_t*)tmp, t.rows, t.row0, t.w);
        else if (dt == LQ8_DTYPE_F32) st = launch_quantize_weight_f32(ctx->stream, (const float*)tmp, t.rows, t.row0, t.w);
        else st = launch_quantize_weight_bf16(ctx->stream, (const uint16_t*)tmp, t.rows, t.row0, t.w);
        if (!st) {
            e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) st = hip_fail(e, "tensor repack");
        }
    }
    if (tmp) (void)hipFree(tmp);
    if (st) { release(m); return st; }
    *out = m;
    return LQ8_OK;
}

lq8_status lq8_model_create(lq8_ctx* ctx, const lq8_qwen3_config* cfg, const void* const* tensors, lq8_model** out) {
    return lq8_model_create_typed(ctx, cfg, tensors, nullptr, out);
}

lq8_status lq8_model_create_random(lq8_ctx* ctx, const lq8_qwen3_config* cfg, uint64_t seed, float stddev,
                                   lq8_model** out) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid context handle");
    if (!out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    lq8_status st = validate(cfg);
    if (st) return st;
    LQ8_HIP(hipSetDevice(ctx->device));
    lq8_model* m = new lq8_model();
    registry_add(m);
    if ((st = build_skeleton(ctx, cfg, m))) { release(m); return st; }
    size_t count = lq8_model_tensor_count(cfg);
    for (size_t i = 0; i < count && !st; i++) {
        TensorRef t = tensor_ref(m, i);
        if (t.norm) st = fill_norm(t.norm, t.norm_len, nullptr);
        else st = launch_random_weight(ctx->stream, t.w, t.row0, t.rows, seed, i, stddev);
    }
    if (!st) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) st = hip_fail(e, "random init");
    }
    if (st) { release(m); return st; }
    *out = m;
    return LQ8_OK;
}

lq8_status lq8_model_export_tensor(lq8_model* m, size_t idx, void* host_out) {
    CHECK_M(m);
    if (!host_out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (idx >= lq8_model_tensor_count(&m->c)) return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "tensor index out of range");
    TensorRef t = tensor_ref(m, idx);
    hipStream_t s = m->ctx->stream;
    if (t.norm) {
        LQ8_HIP(hipMemcpyAsync(host_out, t.norm, t.norm_len * sizeof(float), hipMemcpyDeviceToHost, s));
        LQ8_HIP(hipStreamSynchronize(s));
        return LQ8_OK;
    }
    size_t bytes = t.rows * t.w->nb * BLOCK_BYTES;
    void* tmp = nullptr;
    LQ8_HIP(hipMalloc(&tmp, bytes));
    lq8_status st = launch_unpack_aos(s, t.w, t.row0, t.rows, (uint8_t*)tmp);
    hipError_t e = st ? hipSuccess : hipMemcpyAsync(host_out, tmp, bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(tmp);
    if (st) return st;
    if (e != hipSuccess) return hip_fail(e, "tensor export");
    return LQ8_OK;
}

lq8_status lq8_model_clear_kv_cache(lq8_model* m) {
    CHECK_M(m);
    m->kv_len = 0;
    return LQ8_OK;
}

lq8_status lq8_model_forward(lq8_model* m, const uint32_t* ids, size_t n, size_t offset, float* logits) {
    CHECK_M(m);
    if (!ids || n == 0) return fail(LQ8_ERR_INVALID_ARG, "input_ids cannot be empty");
    if (offset != m->kv_len)
        return fail(LQ8_ERR_INVALID_ARG, "offset must equal the number of cached positions");
    if (offset + n > m->c.max_positions) return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "positions exceed max_positions");
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= m->c.vocab_size) return fail(LQ8_ERR_INVALID_ARG, "token id out of range for vocab_size");
    LQ8_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    lq8_status st;
    if ((st = ensure_ids(m, n))) return st;
    LQ8_HIP(hipMemcpyAsync(m->d_ids, ids, n * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    if (n == 1) {
        st = enqueue_decode(m, m->d_ids, nullptr, (int)offset);
    } else {
        if ((st = ensure_prefill(m, n))) return st;
        st = enqueue_prefill(m, (int)n, (int)offset);
    }
    if (st) return st;
    if (logits)
        LQ8_HIP(hipMemcpyAsync(logits, m->logits, m->c.vocab_size * sizeof(float), hipMemcpyDeviceToHost, s));
    LQ8_HIP(hipStreamSynchronize(s));
    m->kv_len = offset + n;
    return LQ8_OK;
}

lq8_status lq8_model_forward_with_intermediates(lq8_model* m, const uint32_t* ids, size_t n, size_t offset,
                                                float* hidden, float* final_norm, float* logits) {
    CHECK_M(m);
    if (!ids || n == 0) return fail(LQ8_ERR_INVALID_ARG, "input_ids cannot be empty");
    if (!hidden || !final_norm) return fail(LQ8_ERR_INVALID_ARG, "null output pointer");
    if (offset != m->kv_len) return fail(LQ8_ERR_INVALID_ARG, "offset must equal the number of cached positions");
    if (offset + n > m->c.max_positions) return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "positions exceed max_positions");
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= m->c.vocab_size) return fail(LQ8_ERR_INVALID_ARG, "token id out of range for vocab_size");
    LQ8_HIP(hipSetDevice(m->ctx->device));
    hipStream_t s = m->ctx->stream;
    const int Hd = (int)m->c.hidden_size;
    lq8_status st;
    if ((st = ensure_ids(m, n)) || (st = ensure_prefill(m, n))) return st;
    LQ8_HIP(hipMemcpyAsync(m->d_ids, ids, n * sizeof(uint32_t), hipMemcpyHostToDevice, s));
    const float* last;
    if (n == 1) {
        st = enqueue_decode(m, m->d_ids, nullptr, (int)offset, hidden, m->P_h);
        last = m->P_h;
    } else {
        st = enqueue_prefill(m, (int)n, (int)offset, hidden);
        last = m->P_h;
    }
    if (st) return st;
    // final norm of every position (src/model.rs:194)
    if ((st = launch_rms_norm_rows(s, last, m->final_norm, (int)n, Hd, m->c.rms_norm_eps, m->P_x))) return st;
    LQ8_HIP(hipMemcpyAsync(final_norm, m->P_x, n * Hd * sizeof(float), hipMemcpyDeviceToHost, s));
    if (logits)
        LQ8_HIP(hipMemcpyAsync(logits, m->logits, m->c.vocab_size * sizeof(float), hipMemcpyDeviceToHost, s));
    LQ8_HIP(hipStreamSynchronize(s));
    m->kv_len = offset + n;
    return LQ8_OK;
}

lq8_status lq8_generate_greedy(lq8_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                               uint32_t* out_tokens, lq8_gen_stats* stats) {
    CHECK_M(m);
    return run_generate(m, prompt, n_prompt, max_new, nullptr, false, out_tokens, stats);
}

lq8_status lq8_model_persist_picks(lq8_model* m, uint32_t back, float* values, uint32_t* indices, size_t capacity,
                                   size_t* count) {
    CHECK_M(m);
    if (!values || !indices || !count) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (back > 1) return fail(LQ8_ERR_INVALID_ARG, "back must be 0 (the last step) or 1 (the step before)");
    if (!m->persist_wg || (int)back >= m->last_steps)
        return fail(LQ8_ERR_INVALID_ARG, "no such step in the last persistent decode launch");
    *count = (size_t)m->persist_wg;
    if (capacity < (size_t)m->persist_wg) return fail(LQ8_ERR_SHAPE_MISMATCH, "capacity below the workgroup count");
    LQ8_HIP(hipSetDevice(m->ctx->device));
    const unsigned tag = m->tag - 1 - back;
    const size_t P = (size_t)m->persist_wg;
    std::vector<uint64_t> w(2 * P);
    LQ8_HIP(hipStreamSynchronize(m->ctx->stream));
    LQ8_HIP(hipMemcpy(w.data(), m->h_pargs.argb + (size_t)(tag & 1) * 2 * P, 2 * P * sizeof(uint64_t),
                      hipMemcpyDeviceToHost));
    for (size_t i = 0; i < 2 * P; i++)
        if ((unsigned)(w[i] >> 32) != tag) return fail(LQ8_ERR_INVALID_ARG, "that step's picks are not recorded");
    for (size_t i = 0; i < P; i++) {
        const uint32_t vb = (uint32_t)w[2 * i], ib = (uint32_t)w[2 * i + 1];
        std::memcpy(&values[i], &vb, sizeof(float));
        indices[i] = ib;
    }
    return LQ8_OK;
}

lq8_status lq8_generate_ex(lq8_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                           const lq8_sampling* cfg, const uint32_t* eos_ids, size_t n_eos, uint32_t flags,
                           uint32_t* out_tokens, size_t* n_out, lq8_gen_stats* stats) {
    CHECK_M(m);
    if (n_eos && !eos_ids) return fail(LQ8_ERR_INVALID_ARG, "eos_ids is null");
    if (!n_out) return fail(LQ8_ERR_INVALID_ARG, "n_out is null");
    if (flags & ~(uint32_t)LQ8_GEN_FEED_FIRST_TOKEN) return fail(LQ8_ERR_INVALID_ARG, "unknown generation flag");
    const bool feed_first = (flags & LQ8_GEN_FEED_FIRST_TOKEN) != 0;
    SampleCfg sc;
    lq8_status st = check_sampling(cfg, &sc);
    if (st) return st;
    // temperature 0 without a penalty is the greedy rule exactly
    const bool greedy = sc.temperature == 0.0f && std::fabs(sc.penalty - 1.0f) < 1e-6f;
    if (!greedy && !sample_vocab_ok(m->c.vocab_size))
        return fail(LQ8_ERR_INVALID_ARG, "sampling: vocabulary above 2^20");
    if ((st = run_generate(m, prompt, n_prompt, max_new, greedy ? nullptr : &sc, feed_first, out_tokens, stats)))
        return st;
    // the first EOS ends the generation (kept); the cache as after the early stop
    size_t n = max_new;
    for (size_t t = 0; t < max_new && n == max_new; t++)
        for (size_t e = 0; e < n_eos; e++)
            if (out_tokens[t] == eos_ids[e]) {
                n = t + 1;
                break;
            }
    m->kv_len = n_prompt + n - 1;
    *n_out = n;
    return LQ8_OK;
}

lq8_status lq8_generate(lq8_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                        const lq8_sampling* cfg, const uint32_t* eos_ids, size_t n_eos, uint32_t* out_tokens,
                        size_t* n_out, lq8_gen_stats* stats) {
    return lq8_generate_ex(m, prompt, n_prompt, max_new, cfg, eos_ids, n_eos, 0, out_tokens, n_out, stats);
}

lq8_status lq8_model_free(lq8_model* m) {
    CHECK_M(m);
    (void)hipStreamSynchronize(m->ctx->stream);
    release(m);
    return LQ8_OK;
}

}  // extern "C"
