// moe.hip -- Qwen3-MoE decoder layers (Qwen3-30B-A3B style) for decode steps
// of a batch of independent sequences: router, grouped expert GEMVs,
// expert combine, and the layer runtime behind the lq8_moe_* C ABI.
//
// Per layer (T sequences, one token each):
//   qkv   = [q|k|v](RmsNorm(h))               GEMV (T = 1) / W8A8 GEMM (T > 1)
//   part  = attention segments per sequence    (q/k norm, RoPE, KV append)
//   h2    = h + o(attention(part))             GEMV with the combine fused (T = 1),
//                                              combine fused into the activation
//                                              quantizer + W8A8 GEMM (T > 1)
//   route = top_k of softmax(scores)           all layers in one launch before the first
//                                              layer (scores are inputs); expert lists on the device
//   act   = silu(gate_e x) * up_e x, x = RmsNorm(h2)   grouped multi-vector GEMV over the
//                                              routed experts (gate and up tiles in one workgroup)
//   eo    = down_e(act)                        grouped multi-vector GEMV
//   h     = h2 + sum_e w_e * eo_e              ascending expert index
// The attention projections follow Linear::forward over the [T, hidden]
// input (src/attention.rs:101-136): the W8A32 GEMV for one token, the W8A8
// GEMM (activation rows quantized to Q8_0, per-row and per-element results)
// for more, so a token's result depends on whether it runs alone or in a
// batch, never on the other tokens of the batch.  The experts run the
// single-vector GEMV order per token.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "lq8_internal.h"
#include "lq8_numerics.h"

using namespace lq8;

namespace {

constexpr int MOE_MAX_EXPERTS = 256;
constexpr int MOE_MAX_TOPK = 16;
constexpr int MOE_MAX_BATCH = 64;

struct MoeLayer {
    lq8_weight *qkv = nullptr, *o = nullptr;
    // [E * 2I, H]: expert e's rows from e*2I, gate and up interleaved by 8:
    // its 16-row tile t holds gate rows 8t .. 8t+7, then up rows 8t .. 8t+7
    // (so one tile gives silu(gate) * up of 8 rows)
    lq8_weight *gu = nullptr;
    lq8_weight *down = nullptr;  // [E * H, I]: expert e rows e*H ..
    float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

}  // namespace

struct lq8_moe {
    lq8_ctx* ctx = nullptr;
    lq8_moe_config c{};
    size_t QD = 0, KD = 0, QKV = 0;
    int cmax = 0;
    std::vector<MoeLayer> layers;
    float *cos_t = nullptr, *sin_t = nullptr;
    float *kc = nullptr, *vc = nullptr;  // [layer][seq][kv_head][max_pos][128]
    float *h2 = nullptr, *qkv = nullptr, *apart = nullptr;
    float* xn = nullptr;  // [max_batch][hidden]: RmsNorm rows (batched decode)
    int8_t* xq = nullptr;    // activation operand of the batched GEMMs (codes)
    uint32_t* xs = nullptr;  // and its scales
    float *gu = nullptr;  // [max_batch * top_k][expert_intermediate]: silu(gate) * up per slot
    float *eo = nullptr;  // [max_batch * top_k][hidden]: expert outputs per slot
    uint32_t* rids = nullptr;  // [layer][max_batch][top_k]
    float* rw = nullptr;
    int *n_act = nullptr, *act_e = nullptr, *vbeg = nullptr, *vcnt = nullptr;  // per layer: [layer], [layer][E]
    int* slots = nullptr;                                                      // [layer][max_batch * top_k]
    float *hid_tmp = nullptr, *scores_tmp = nullptr;
    int* pos_tmp = nullptr;
    size_t last_T = 0;
};

namespace {

// ---- router ------------------------------------------------------------------
// One workgroup of 16 waves for the batch.  Wave w routes tokens w, w + 16,
// ...: lane l holds scores l, l + 64, ...; m = max (exact in any order),
// e = exp(s - m), S = SUM64(e) (lane l adds its entries in order, then the
// xor fold), p = e / S.  An entry's rank is the number of entries with a
// larger p or an equal p and a lower index; ranks below top_k are chosen, in
// rank order; weights p_r / (((p_0 + p_1) + p_2) + ...).  Then the routed
// (token, rank) slots t * top_k + r are counted per expert, the active
// experts numbered by descending vector count, then ascending index (n_act,
// act_e, vbeg, vcnt; the expert GEMVs' workgroups follow that order), and
// each slot placed in its expert's list (slots, by ascending expert).  The order inside one expert's
// list is whatever the atomics give: every slot is computed on its own, so
// results do not depend on it.
constexpr int ROUTE_WAVES = 16;
struct RouteArgs {
    const float* scores;  // [layers][T][E]
    int T, E, K, B;       // B: per-layer stride of the slot tables (max_batch)
    uint32_t* rids;       // [layers][B][K]
    float* rw;            // [layers][B][K]
    int* n_act;           // [layers]
    int* act_e;           // [layers][E]
    int* vbeg;            // [layers][E]
    int* vcnt;            // [layers][E]
    int* slots;           // [layers][B * K]
};
__global__ __launch_bounds__(64 * ROUTE_WAVES) void k_moe_route(RouteArgs ra) {
    __shared__ float4 sp4[ROUTE_WAVES][MOE_MAX_EXPERTS / 4];
    __shared__ float selp[ROUTE_WAVES][MOE_MAX_TOPK];
    __shared__ int sid[MOE_MAX_BATCH * MOE_MAX_TOPK];
    __shared__ int cnt[MOE_MAX_EXPERTS], beg[MOE_MAX_EXPERTS], fill[MOE_MAX_EXPERTS];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const float NEG = -__builtin_huge_valf();
    const int l = blockIdx.x, T = ra.T, E = ra.E, K = ra.K;
    const float* __restrict__ scores = ra.scores + (size_t)l * T * E;
    uint32_t* __restrict__ rids = ra.rids + (size_t)l * ra.B * K;
    float* __restrict__ rw = ra.rw + (size_t)l * ra.B * K;
    int* __restrict__ act_e = ra.act_e + (size_t)l * E;
    int* __restrict__ vbeg = ra.vbeg + (size_t)l * E;
    int* __restrict__ vcnt = ra.vcnt + (size_t)l * E;
    int* __restrict__ slots = ra.slots + (size_t)l * ra.B * K;
    float* sp = (float*)sp4[wave];
    const int E16 = (E + 15) & ~15;  // the rank loop reads 16 entries at a time; padding is -inf
    for (int e = tid; e < E; e += 64 * ROUTE_WAVES) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    for (int t = wave; t < T; t += ROUTE_WAVES) {
        float p[4];
        float m = NEG;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = lane + 64 * j;
            p[j] = i < E ? scores[(size_t)t * E + i] : NEG;
            m = fmaxf(m, p[j]);
        }
        m = fmaxf(m, lane_xor<32>(m));
        m = fmaxf(m, lane_xor<16>(m));
        m = fmaxf(m, lane_xor<8>(m));
        m = fmaxf(m, lane_xor<4>(m));
        m = fmaxf(m, lane_xor<2>(m));
        m = fmaxf(m, lane_xor<1>(m));
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (lane + 64 * j < E) {
                p[j] = expf_cr(p[j] - m);
                acc = acc + p[j];
            }
        }
        acc = wave_sum64(acc);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = lane + 64 * j;
            if (i < E) p[j] = __fdiv_rn(p[j], acc);
            if (i < E16) sp[i] = p[j];  // NEG past E
        }
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        // rank = entries with a larger p, or an equal p and a lower index
        int rank[4] = {0, 0, 0, 0};
        for (int i0 = 0; i0 < E16; i0 += 16) {
            float4 q4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) q4[u] = sp4[wave][(i0 >> 2) + u];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float q[4] = {q4[u].x, q4[u].y, q4[u].z, q4[u].w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int i2 = i0 + 4 * u + c;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int i = lane + 64 * j;
                        rank[j] += (q[c] > p[j] || (q[c] == p[j] && i2 < i)) ? 1 : 0;
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = lane + 64 * j;
            if (i < E && rank[j] < K) {
                selp[wave][rank[j]] = p[j];
                rids[t * K + rank[j]] = (uint32_t)i;
                sid[t * K + rank[j]] = i;
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        float pk[MOE_MAX_TOPK];
#pragma unroll
        for (int r = 0; r < MOE_MAX_TOPK; r++) pk[r] = r < K ? selp[wave][r] : 0.0f;
        float tot = 0.0f;
#pragma unroll
        for (int r = 0; r < MOE_MAX_TOPK; r++)
            if (r < K) tot = tot + pk[r];
        if (lane < K) rw[t * K + lane] = __fdiv_rn(selp[wave][lane], tot);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    for (int s = tid; s < T * K; s += 64 * ROUTE_WAVES) atomicAdd(&cnt[sid[s]], 1);
    __syncthreads();
    if (wave == 0) {
        // ascending scan over the experts: lane l owns experts 4l .. 4l + 3
        int c[4], nz = 0, tot = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = 4 * lane + q;
            c[q] = e < E ? cnt[e] : 0;
            tot += c[q];
            nz += c[q] > 0;
        }
        int ptot = tot, pnz = nz;  // inclusive prefix over lanes
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int a1 = __shfl_up(ptot, d, 64), a2 = __shfl_up(pnz, d, 64);
            if (lane >= d) { ptot += a1; pnz += a2; }
        }
        int off = ptot - tot;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = 4 * lane + q;
            if (e < E) {
                beg[e] = off;
                if (c[q]) {
                    // problem number: experts with more vectors first (then
                    // ascending index), so the longest workgroups start first
                    int j = 0;
                    for (int f = 0; f < E; f++) {
                        const int cf = cnt[f];
                        j += cf > c[q] || (cf == c[q] && f < e);
                    }
                    act_e[j] = e;
                    vbeg[j] = off;
                    vcnt[j] = c[q];
                }
                off += c[q];
            }
        }
        if (lane == 63) ra.n_act[l] = pnz;
    }
    __syncthreads();
    for (int s = tid; s < T * K; s += 64 * ROUTE_WAVES) {
        const int e = sid[s];
        slots[beg[e] + atomicAdd(&fill[e], 1)] = s;
    }
}

// ---- expert combine -----------------------------------------------------------
// out[t][i] = h2[t][i] + acc, acc = ((0 + w_a * eo_a) + w_b * eo_b) + ... over
// the token's experts in ascending expert index (products rounded, then added).
__global__ __launch_bounds__(256) void k_moe_combine(const float* __restrict__ h2, const float* __restrict__ eo,
                                                     const uint32_t* __restrict__ rids, const float* __restrict__ rw,
                                                     int K, int H, float* __restrict__ out) {
    __shared__ int order[MOE_MAX_TOPK];  // ranks in ascending expert index
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (threadIdx.x < K) {
        const uint32_t me = rids[t * K + threadIdx.x];
        int below = 0;
        for (int r = 0; r < K; r++) below += rids[t * K + r] < me;
        order[below] = threadIdx.x;  // expert ids of a token are distinct
    }
    __syncthreads();
    if (i >= H) return;
    float wv[MOE_MAX_TOPK], ev[MOE_MAX_TOPK];
#pragma unroll
    for (int q = 0; q < MOE_MAX_TOPK; q++) {
        const int slot = t * K + order[q < K ? q : 0];
        wv[q] = rw[slot];
        ev[q] = eo[(size_t)slot * H + i];
    }
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < MOE_MAX_TOPK; q++)
        if (q < K) acc = acc + wv[q] * ev[q];
    out[(size_t)t * H + i] = h2[(size_t)t * H + i] + acc;
}

template <typename T>
lq8_status dalloc(T** p, size_t count) {
    *p = nullptr;
    if (!count) return LQ8_OK;
    hipError_t e = hipMalloc((void**)p, count * sizeof(T));
    if (e != hipSuccess) {
        *p = nullptr;
        return e == hipErrorOutOfMemory ? fail(LQ8_ERR_OUT_OF_MEMORY, "device allocation failed")
                                        : hip_fail(e, "hipMalloc");
    }
    return LQ8_OK;
}

lq8_status validate(const lq8_moe_config* c) {
    if (!c) return fail(LQ8_ERR_INVALID_ARG, "null config");
    if (c->head_dim != 128 || !attention_supported((int)c->num_heads, (int)c->num_kv_heads, (int)c->head_dim))
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: head_dim 128 and num_heads / num_kv_heads <= 16 required");
    if (c->hidden_size == 0 || c->hidden_size % 32 || c->hidden_size > GEMV_MAX_K)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: hidden_size must be a multiple of 32 up to 12288");
    if ((size_t)c->num_heads * c->head_dim > GEMV_MAX_K)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: num_heads * head_dim above 12288");
    if (c->expert_intermediate_size == 0 || c->expert_intermediate_size % 32 || c->expert_intermediate_size > GEMV_MAX_K)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: expert_intermediate_size must be a multiple of 32 up to 12288");
    if (c->num_experts == 0 || c->num_experts > MOE_MAX_EXPERTS)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: num_experts must be 1..256");
    if (c->top_k == 0 || c->top_k > c->num_experts || c->top_k > MOE_MAX_TOPK)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: top_k must be 1..min(num_experts, 16)");
    if (c->max_batch == 0 || c->max_batch > MOE_MAX_BATCH)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: max_batch must be 1..64");
    if (c->max_positions == 0 || c->max_positions > (1u << 20))
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: max_positions must be 1..1048576");
    if (c->num_layers == 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: num_layers must be positive");
    return LQ8_OK;
}

void release(lq8_moe* m) {
    if (!m) return;
    registry_remove(m);
    auto F = [](void* p) { if (p) (void)hipFree(p); };
    for (auto& L : m->layers) {
        weight_release(L.qkv); weight_release(L.o); weight_release(L.gu); weight_release(L.down);
        F(L.in_norm); F(L.post_norm); F(L.q_norm); F(L.k_norm);
    }
    F(m->cos_t); F(m->sin_t); F(m->kc); F(m->vc);
    F(m->h2); F(m->xn); F(m->xq); F(m->xs); F(m->qkv); F(m->apart); F(m->gu); F(m->eo);
    F(m->rids); F(m->rw); F(m->n_act); F(m->act_e); F(m->vbeg); F(m->vcnt); F(m->slots);
    F(m->hid_tmp); F(m->scores_tmp); F(m->pos_tmp);
    delete m;
}

lq8_status build_skeleton(lq8_ctx* ctx, const lq8_moe_config* c, lq8_moe* m) {
    m->ctx = ctx;
    m->c = *c;
    const size_t H = c->hidden_size, I = c->expert_intermediate_size, hd = c->head_dim, P = c->max_positions;
    const size_t E = c->num_experts, B = c->max_batch, K = c->top_k, NL = c->num_layers;
    m->QD = (size_t)c->num_heads * hd;
    m->KD = (size_t)c->num_kv_heads * hd;
    m->QKV = m->QD + 2 * m->KD;
    m->cmax = (int)((P + ATT_SEG - 1) / ATT_SEG);
    lq8_status st;
    m->layers.resize(NL);
    for (auto& L : m->layers) {
        if ((st = weight_alloc(ctx, m->QKV, H, &L.qkv)) || (st = weight_alloc(ctx, H, m->QD, &L.o)) ||
            (st = weight_alloc(ctx, E * 2 * I, H, &L.gu)) || (st = weight_alloc(ctx, E * H, I, &L.down)))
            return st;
        if ((st = dalloc(&L.in_norm, H)) || (st = dalloc(&L.post_norm, H)) || (st = dalloc(&L.q_norm, hd)) ||
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
    const size_t kv = NL * B * c->num_kv_heads * P * hd;
    if ((st = dalloc(&m->kc, kv)) || (st = dalloc(&m->vc, kv))) return st;
    LQ8_HIP(hipMemset(m->kc, 0, kv * sizeof(float)));
    LQ8_HIP(hipMemset(m->vc, 0, kv * sizeof(float)));
    if ((st = dalloc(&m->h2, B * H)) || (st = dalloc(&m->xn, B * H)) || (st = dalloc(&m->qkv, B * m->QKV)) ||
        (st = dalloc(&m->apart, B * m->cmax * c->num_heads * ATT_PART_STRIDE)) ||
        (st = dalloc(&m->gu, B * K * I)) || (st = dalloc(&m->eo, B * K * H)) ||
        (st = dalloc(&m->rids, NL * B * K)) || (st = dalloc(&m->rw, NL * B * K)) || (st = dalloc(&m->n_act, NL)) ||
        (st = dalloc(&m->act_e, NL * E)) || (st = dalloc(&m->vbeg, NL * E)) || (st = dalloc(&m->vcnt, NL * E)) ||
        (st = dalloc(&m->slots, NL * B * K)) || (st = dalloc(&m->hid_tmp, B * H)) ||
        (st = dalloc(&m->scores_tmp, NL * B * E)) || (st = dalloc(&m->pos_tmp, B)))
        return st;
    const int kmax = (int)std::max(H, m->QD);
    if ((st = dalloc(&m->xq, act_code_bytes((int)B, kmax))) || (st = dalloc(&m->xs, act_scale_bytes((int)B, kmax) / 4)))
        return st;
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

size_t per_layer(const lq8_moe_config* c) { return 8 + 3 * (size_t)c->num_experts; }

struct TensorRef {
    lq8_weight* w = nullptr;
    size_t row0 = 0, rows = 0;
    RowRun rr;  // where the tensor's rows sit in w
    float* norm = nullptr;
    size_t norm_len = 0;
};

TensorRef tensor_ref(lq8_moe* m, size_t idx) {
    TensorRef t;
    const size_t H = m->c.hidden_size, I = m->c.expert_intermediate_size, E = m->c.num_experts;
    const size_t l = idx / per_layer(&m->c), k = idx % per_layer(&m->c);
    MoeLayer& L = m->layers[l];
    switch (k) {
        case 0: t.norm = L.in_norm; t.norm_len = H; return t;
        case 1: t.norm = L.post_norm; t.norm_len = H; return t;
        case 2: t.norm = L.q_norm; t.norm_len = m->c.head_dim; return t;
        case 3: t.norm = L.k_norm; t.norm_len = m->c.head_dim; return t;
        case 4: t.w = L.qkv; t.row0 = 0; t.rows = m->QD; return t;
        case 5: t.w = L.qkv; t.row0 = m->QD; t.rows = m->KD; return t;
        case 6: t.w = L.qkv; t.row0 = m->QD + m->KD; t.rows = m->KD; return t;
        case 7: t.w = L.o; t.rows = H; return t;
        default: break;
    }
    const size_t x = k - 8, e = x % E;
    if (x < 2 * E) {
        // gate (x < E) or up: runs of 8 rows, every 16 rows
        t.w = L.gu;
        t.row0 = e * 2 * I + (x < E ? 0 : 8);
        t.rows = I;
        t.rr.run = 8;
        t.rr.stride = 16;
    }
    else { t.w = L.down; t.row0 = e * H; t.rows = H; }
    return t;
}

lq8_status enqueue_forward(lq8_moe* m, float* d_hidden, const float* d_scores, const int* d_pos, int T) {
    hipStream_t s = m->ctx->stream;
    const lq8_moe_config& c = m->c;
    const int H = (int)c.hidden_size, I = (int)c.expert_intermediate_size, E = (int)c.num_experts, K = (int)c.top_k;
    const int NH = (int)c.num_heads, B = (int)c.max_batch;
    const size_t P = c.max_positions;
    const size_t seq_kv = (size_t)c.num_kv_heads * P * 128, layer_kv = (size_t)B * seq_kv;
    const size_t part_stride = (size_t)m->cmax * NH * ATT_PART_STRIDE;
    const float scale = 1.0f / std::sqrt((float)c.head_dim);
    const int max_probs = std::min(E, T * K);
    lq8_status st;
    // the router reads only the given scores: every layer's routing in one launch
    RouteArgs ra{d_scores, T, E, K, B, m->rids, m->rw, m->n_act, m->act_e, m->vbeg, m->vcnt, m->slots};
    hipLaunchKernelGGL(k_moe_route, dim3((unsigned)m->layers.size()), dim3(64 * ROUTE_WAVES), 0, s, ra);
    LQ8_HIP(hipGetLastError());
    bool prequant = false;  // T > 1: the previous layer's combine wrote this layer's q|k|v operand
    for (size_t l = 0; l < m->layers.size(); l++) {
        MoeLayer& L = m->layers[l];
        int* n_act = m->n_act + l;
        int* act_e = m->act_e + l * E;
        int* vbeg = m->vbeg + l * E;
        int* vcnt = m->vcnt + l * E;
        int* slots = m->slots + l * (size_t)B * K;
        // input_layernorm + q|k|v.  T = 1: the norm is fused into the GEMV's
        // input staging; T > 1: the norm is fused into the activation
        // quantizer of the GEMM (the operand rms_norm_rows + quantize_act give)
        if (T == 1) {
            GemvArgs g{L.qkv->codes, L.qkv->scales, d_hidden, L.in_norm, m->qkv, nullptr, nullptr, nullptr,
                       (int)m->QKV, H, c.rms_norm_eps};
            if ((st = launch_gemv(s, XS_RMSNORM, EPI_STORE, g))) return st;
        } else {
            if (prequant) {
                // xq / xs already hold RmsNorm(h) of this layer (the previous combine)
            } else if (rms_quantize_supported(H)) {
                if ((st = launch_rms_quantize_act(s, d_hidden, L.in_norm, T, H, c.rms_norm_eps, m->xq, m->xs)))
                    return st;
            } else {
                if ((st = launch_rms_norm_rows(s, d_hidden, L.in_norm, T, H, c.rms_norm_eps, m->xn))) return st;
                if ((st = launch_quantize_act(s, m->xn, T, H, m->xq, m->xs))) return st;
            }
            if ((st = launch_gemm(s, m->xq, m->xs, T, L.qkv, m->qkv, nullptr))) return st;
        }
        // q/k norm, RoPE, KV append, attention per segment, per sequence
        AttnSegLaunch at{m->qkv, L.q_norm, L.k_norm, m->cos_t, m->sin_t, m->kc + l * layer_kv, m->vc + l * layer_kv,
                         m->apart, d_pos, 0, NH, (int)c.num_kv_heads, (int)P, c.rms_norm_eps, scale};
        at.batch = T;
        at.qkv_stride = m->QKV;
        at.kv_stride = seq_kv;
        at.part_stride = part_stride;
        at.head_group = T == 1 ? 2 : 0;  // one sequence: a kv head's query heads over G / 2 workgroups
        if ((st = launch_attention_seg(s, at))) return st;
        // o_proj on the attention output, + residual -> h2
        if (T == 1) {
            GemvArgs g{L.o->codes, L.o->scales, m->apart, nullptr, m->h2, d_hidden, nullptr, nullptr, H, (int)m->QD,
                       0.0f};
            g.d_pos = d_pos;
            g.attn_heads = NH;
            g.attn_cmax = m->cmax;
            if ((st = launch_gemv(s, XS_ATTN, EPI_RESID, g))) return st;
        } else {
            // the segment combine fused into the activation quantizer
            if ((st = launch_attention_combine_quant(s, m->apart, part_stride, d_pos, T, NH, m->cmax, m->xq, m->xs)))
                return st;
            if ((st = launch_gemm(s, m->xq, m->xs, T, L.o, m->h2, d_hidden))) return st;
        }
        uint32_t* rids = m->rids + l * B * K;
        float* rw = m->rw + l * B * K;
        // post_attention_layernorm + gate and up of each routed expert -> silu(gate) * up
        // (the norm fused at T = 1, once per row at T > 1, as above)
        MvArgs g{};
        g.codes = L.gu->codes; g.scales = L.gu->scales; g.rows = 2 * I; g.k = H; g.prob_tiles = 2 * I / TILE_ROWS;
        g.n_prob = n_act; g.prob_id = act_e; g.vec_begin = vbeg; g.vec_count = vcnt; g.slots = slots;
        g.x_stride = H; g.x_div = K; g.y = m->gu; g.y_stride = I; g.max_vec = T;
        if (T == 1 && moe_gate_up1_supported(K, I, H)) {
            // one token: the experts by rank straight from the router's list
            const MoeGateUpArgs gu1{L.gu->codes, L.gu->scales, I, H, 2 * I / TILE_ROWS, rids, K,
                                    m->h2, L.post_norm, c.rms_norm_eps, m->gu, I};
            if ((st = launch_moe_gate_up1(s, gu1))) return st;
        } else if (T == 1) {
            g.x = m->h2;
            g.norm_w = L.post_norm;
            g.eps = c.rms_norm_eps;
            if ((st = launch_gemv_mv(s, XS_RMSNORM, EPI_SWIGLU, g, max_probs, 1))) return st;
        } else {
            if ((st = launch_rms_norm_rows(s, m->h2, L.post_norm, T, H, c.rms_norm_eps, m->xn))) return st;
            g.x = m->xn;
            if ((st = launch_gemv_mv(s, XS_PLAIN, EPI_SWIGLU, g, max_probs, 1))) return st;
        }
        // down of each routed expert; batch 1: fused with the combine
        if (T == 1 && moe_down_combine_supported(K, I)) {
            MoeDownArgs dc{L.down->codes, L.down->scales, H, I, H / TILE_ROWS, rids, rw, K, m->gu, I, m->h2, d_hidden};
            if ((st = launch_moe_down_combine(s, dc))) return st;
            continue;
        }
        MvArgs d{};
        d.codes = L.down->codes; d.scales = L.down->scales; d.rows = H; d.k = I; d.prob_tiles = H / TILE_ROWS;
        d.n_prob = n_act; d.prob_id = act_e; d.vec_begin = vbeg; d.vec_count = vcnt; d.slots = slots;
        d.x = m->gu; d.x_stride = I; d.x_div = 1; d.y = m->eo; d.y_stride = H; d.max_vec = T;
        if ((st = launch_gemv_mv(s, XS_PLAIN, EPI_STORE, d, max_probs, 1))) return st;
        // h = h2 + experts (ascending expert index); below the last layer fused
        // with the next layer's input_layernorm + activation quantize
        prequant = T > 1 && l + 1 < m->layers.size() && combine_rms_quant_supported(K, H);
        if (prequant) {
            if ((st = launch_combine_rms_quant(s, m->h2, m->eo, rids, rw, K, T, H, m->layers[l + 1].in_norm,
                                               c.rms_norm_eps, d_hidden, m->xq, m->xs)))
                return st;
            continue;
        }
        hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((H + 255) / 256), (unsigned)T), dim3(256), 0, s, m->h2, m->eo,
                           rids, rw, K, H, d_hidden);
        LQ8_HIP(hipGetLastError());
    }
    return LQ8_OK;
}

lq8_status upload_table(lq8_moe* m, const void* const* tensors) {
    const size_t count = m->layers.size() * per_layer(&m->c);
    void* tmp = nullptr;
    size_t tmp_cap = 0;
    lq8_status st = LQ8_OK;
    for (size_t i = 0; i < count && !st; i++) {
        TensorRef t = tensor_ref(m, i);
        if (t.norm) { st = fill_norm(t.norm, t.norm_len, (const float*)tensors[i]); continue; }
        const size_t bytes = t.rows * t.w->nb * BLOCK_BYTES;
        if (bytes > tmp_cap) {
            if (tmp) (void)hipFree(tmp);
            tmp = nullptr;
            hipError_t e = hipMalloc(&tmp, bytes);
            if (e != hipSuccess) { st = hip_fail(e, "staging"); break; }
            tmp_cap = bytes;
        }
        hipError_t e = hipMemcpy(tmp, tensors[i], bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) { st = hip_fail(e, "tensor upload"); break; }
        st = launch_repack_aos(m->ctx->stream, (const uint8_t*)tmp, t.rows, t.row0, t.w, t.rr);
        if (!st) {
            e = hipStreamSynchronize(m->ctx->stream);
            if (e != hipSuccess) st = hip_fail(e, "tensor repack");
        }
    }
    if (tmp) (void)hipFree(tmp);
    return st;
}

}  // namespace

#define CHECK_MOE(m) \
    if (!registry_has(m)) return fail(LQ8_ERR_INVALID_ARG, "invalid or released MoE handle")

extern "C" {

size_t lq8_moe_tensor_count(const lq8_moe_config* cfg) { return cfg ? per_layer(cfg) * cfg->num_layers : 0; }

lq8_status lq8_moe_tensor_bytes(const lq8_moe_config* c, size_t idx, size_t* bytes) {
    if (!c || !bytes) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (idx >= lq8_moe_tensor_count(c)) return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "tensor index out of range");
    const size_t H = c->hidden_size, I = c->expert_intermediate_size, hd = c->head_dim, E = c->num_experts;
    const size_t QD = (size_t)c->num_heads * hd, KD = (size_t)c->num_kv_heads * hd;
    auto q8 = [](size_t r, size_t k) { return r * (k / 32) * 34; };
    const size_t k = idx % per_layer(c);
    switch (k) {
        case 0: case 1: *bytes = H * 4; return LQ8_OK;
        case 2: case 3: *bytes = hd * 4; return LQ8_OK;
        case 4: *bytes = q8(QD, H); return LQ8_OK;
        case 5: case 6: *bytes = q8(KD, H); return LQ8_OK;
        case 7: *bytes = q8(H, QD); return LQ8_OK;
        default: break;
    }
    *bytes = k - 8 < 2 * E ? q8(I, H) : q8(H, I);
    return LQ8_OK;
}

lq8_status lq8_moe_create(lq8_ctx* ctx, const lq8_moe_config* cfg, const void* const* tensors, lq8_moe** out) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid context handle");
    if (!tensors || !out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    lq8_status st = validate(cfg);
    if (st) return st;
    const size_t count = lq8_moe_tensor_count(cfg);
    for (size_t i = 0; i < count; i++)
        if (!tensors[i]) return fail(LQ8_ERR_INVALID_ARG, "null tensor in table");
    LQ8_HIP(hipSetDevice(ctx->device));
    lq8_moe* m = new lq8_moe();
    registry_add(m);
    if ((st = build_skeleton(ctx, cfg, m)) || (st = upload_table(m, tensors))) { release(m); return st; }
    *out = m;
    return LQ8_OK;
}

lq8_status lq8_moe_create_random(lq8_ctx* ctx, const lq8_moe_config* cfg, uint64_t seed, float stddev,
                                 lq8_moe** out) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid context handle");
    if (!out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    lq8_status st = validate(cfg);
    if (st) return st;
    LQ8_HIP(hipSetDevice(ctx->device));
    lq8_moe* m = new lq8_moe();
    registry_add(m);
    if ((st = build_skeleton(ctx, cfg, m))) { release(m); return st; }
    const size_t count = lq8_moe_tensor_count(cfg);
    for (size_t i = 0; i < count && !st; i++) {
        TensorRef t = tensor_ref(m, i);
        if (t.norm) st = fill_norm(t.norm, t.norm_len, nullptr);
        else st = launch_random_weight(ctx->stream, t.w, t.row0, t.rows, seed, i, stddev, t.rr);
    }
    if (!st) {
        hipError_t e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) st = hip_fail(e, "random init");
    }
    if (st) { release(m); return st; }
    *out = m;
    return LQ8_OK;
}

lq8_status lq8_moe_export_tensor(lq8_moe* m, size_t idx, void* host_out) {
    CHECK_MOE(m);
    if (!host_out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (idx >= lq8_moe_tensor_count(&m->c)) return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "tensor index out of range");
    TensorRef t = tensor_ref(m, idx);
    hipStream_t s = m->ctx->stream;
    if (t.norm) {
        LQ8_HIP(hipMemcpyAsync(host_out, t.norm, t.norm_len * sizeof(float), hipMemcpyDeviceToHost, s));
        LQ8_HIP(hipStreamSynchronize(s));
        return LQ8_OK;
    }
    const size_t bytes = t.rows * t.w->nb * BLOCK_BYTES;
    void* tmp = nullptr;
    LQ8_HIP(hipMalloc(&tmp, bytes));
    lq8_status st = launch_unpack_aos(s, t.w, t.row0, t.rows, (uint8_t*)tmp, t.rr);
    hipError_t e = hipSuccess;
    if (!st) e = hipMemcpyAsync(host_out, tmp, bytes, hipMemcpyDeviceToHost, s);
    if (!st && e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(tmp);
    if (st) return st;
    if (e != hipSuccess) return hip_fail(e, "export tensor");
    return LQ8_OK;
}

lq8_status lq8_moe_weight_bytes(lq8_moe* m, size_t* bytes) {
    CHECK_MOE(m);
    if (!bytes) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    size_t total = 0;
    const size_t count = lq8_moe_tensor_count(&m->c);
    for (size_t i = 0; i < count; i++) {
        TensorRef t = tensor_ref(m, i);
        if (t.w) total += t.rows * t.w->nb * BLOCK_BYTES;
    }
    *bytes = total;
    return LQ8_OK;
}

lq8_status lq8_moe_forward_device(lq8_moe* m, float* d_hidden, const float* d_scores, const int32_t* d_pos, size_t T) {
    CHECK_MOE(m);
    if (!d_hidden || !d_scores || !d_pos) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (T == 0 || T > m->c.max_batch) return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: T must be 1..max_batch");
    if (((uintptr_t)d_hidden & 15) != 0) return fail(LQ8_ERR_INVALID_ARG, "hidden must be 16-byte aligned");
    lq8_status st = enqueue_forward(m, d_hidden, d_scores, d_pos, (int)T);
    if (st) return st;
    m->last_T = T;
    return LQ8_OK;
}

lq8_status lq8_moe_forward(lq8_moe* m, float* hidden, const float* scores, const int32_t* pos, size_t T) {
    CHECK_MOE(m);
    if (!hidden || !scores || !pos) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (T == 0 || T > m->c.max_batch) return fail(LQ8_ERR_SHAPE_MISMATCH, "moe: T must be 1..max_batch");
    for (size_t t = 0; t < T; t++)
        if (pos[t] < 0 || (uint32_t)pos[t] >= m->c.max_positions)
            return fail(LQ8_ERR_DIM_OUT_OF_RANGE, "moe: position outside the KV cache");
    hipStream_t s = m->ctx->stream;
    const size_t H = m->c.hidden_size, E = m->c.num_experts, NL = m->c.num_layers;
    LQ8_HIP(hipMemcpyAsync(m->hid_tmp, hidden, T * H * sizeof(float), hipMemcpyHostToDevice, s));
    LQ8_HIP(hipMemcpyAsync(m->scores_tmp, scores, NL * T * E * sizeof(float), hipMemcpyHostToDevice, s));
    LQ8_HIP(hipMemcpyAsync(m->pos_tmp, pos, T * sizeof(int32_t), hipMemcpyHostToDevice, s));
    lq8_status st = enqueue_forward(m, m->hid_tmp, m->scores_tmp, m->pos_tmp, (int)T);
    if (st) return st;
    m->last_T = T;
    LQ8_HIP(hipMemcpyAsync(hidden, m->hid_tmp, T * H * sizeof(float), hipMemcpyDeviceToHost, s));
    LQ8_HIP(hipStreamSynchronize(s));
    return LQ8_OK;
}

lq8_status lq8_moe_routing(lq8_moe* m, uint32_t* experts, float* weights) {
    CHECK_MOE(m);
    if (!experts || !weights) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    const size_t B = m->c.max_batch, K = m->c.top_k, T = m->last_T;
    hipStream_t s = m->ctx->stream;
    for (size_t l = 0; l < m->layers.size(); l++) {
        LQ8_HIP(hipMemcpyAsync(experts + l * T * K, m->rids + l * B * K, T * K * sizeof(uint32_t),
                               hipMemcpyDeviceToHost, s));
        LQ8_HIP(hipMemcpyAsync(weights + l * T * K, m->rw + l * B * K, T * K * sizeof(float), hipMemcpyDeviceToHost, s));
    }
    LQ8_HIP(hipStreamSynchronize(s));
    return LQ8_OK;
}

lq8_status lq8_moe_clear_kv_cache(lq8_moe* m) {
    CHECK_MOE(m);
    const size_t kv = (size_t)m->c.num_layers * m->c.max_batch * m->c.num_kv_heads * m->c.max_positions * 128;
    LQ8_HIP(hipMemsetAsync(m->kc, 0, kv * sizeof(float), m->ctx->stream));
    LQ8_HIP(hipMemsetAsync(m->vc, 0, kv * sizeof(float), m->ctx->stream));
    LQ8_HIP(hipStreamSynchronize(m->ctx->stream));
    return LQ8_OK;
}

lq8_status lq8_moe_free(lq8_moe* m) {
    CHECK_MOE(m);
    (void)hipStreamSynchronize(m->ctx->stream);
    release(m);
    return LQ8_OK;
}

}  // extern "C"
