// model_kernels.hip -- decoder kernels around the Q8_0 linears (gfx950).
//
// Orders follow the CPU oracle exactly:
//   SUM64   lane l (of one 64-lane wave) accumulates elements l, l+64, ... from
//           0; the partials fold at distances 32, 16, 8, 4, 2, 1.  Used for the
//           RMSNorm sum of squares and the softmax denominator.
//   scores  q.k sequential over head_dim (src/tensor.rs:2846-2915), then
//           times 1/sqrt(head_dim).
//   p.v     sequential over positions for each output dimension.
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

__device__ __forceinline__ float wave_sum64(float a) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) a = a + __shfl_xor(a, d, 64);
    return a;
}

// q/k RmsNorm per head (src/attention.rs:350-358), RoPE (src/rope.rs:270-297),
// KV-cache append (src/attention.rs:507-559, without the re-copy).
// grid (n, num_heads + num_kv_heads), block 64.
__global__ __launch_bounds__(64) void k_qk_rope_kv(QkRopeLaunch a) {
    const int i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int hd = a.head_dim, R = hd / 2, per = hd / 64;
    const int QD = a.num_heads * hd, KD = a.num_kv_heads * hd, row = QD + 2 * KD;
    const int pos = (a.d_pos ? *a.d_pos : a.pos_base) + i;
    const bool isq = h < a.num_heads;
    const float* src = a.qkv + (size_t)i * row + (isq ? h * hd : QD + (h - a.num_heads) * hd);
    const float* w = isq ? a.q_norm : a.k_norm;
    float xb[8], y[8];
    float acc = 0.0f;
    for (int t = 0; t < per; t++) {
        float v = bf16_round(src[lane + 64 * t]);
        xb[t] = v;
        acc = acc + v * v;
    }
    acc = wave_sum64(acc);
    const float mean = __fdiv_rn(acc, (float)hd);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(mean + a.eps));
    for (int t = 0; t < per; t++) y[t] = bf16_round((xb[t] * inv) * bf16_round(w[lane + 64 * t]));
    const float* cs = a.cos_t + (size_t)pos * R;
    const float* sn = a.sin_t + (size_t)pos * R;
    const int kvh = h - a.num_heads;
    for (int t = 0; t < per / 2; t++) {
        const int d = lane + 64 * t;
        const float c = cs[d & ~1], s = sn[d & ~1];
        const float x1 = y[t], x2 = y[t + per / 2];
        const float o1 = x1 * c - x2 * s;
        const float o2 = x2 * c + x1 * s;
        if (isq) {
            float* q = a.q_out + (size_t)i * QD + h * hd;
            q[d] = o1;
            q[d + R] = o2;
        } else {
            float* kr = a.k_cache + ((size_t)kvh * a.max_pos + pos) * hd;
            kr[d] = o1;
            kr[d + R] = o2;
        }
    }
    if (!isq) {
        const float* v = a.qkv + (size_t)i * row + QD + KD + kvh * hd;
        float* vc = a.v_cache + ((size_t)kvh * a.max_pos + pos) * hd;
        for (int t = 0; t < per; t++) vc[lane + 64 * t] = v[lane + 64 * t];
    }
}

// One (q head, query row) per workgroup: scores, softmax, p.v
// (src/attention.rs:366-394).  GQA maps q head h to kv head h / groups
// (repeat_kv order, src/attention.rs:442-452).  Query i sees positions
// 0..pos_i (the causal mask of src/causal_mask.rs:128-148; masked terms are
// exact zeros of the softmax and are skipped).
__global__ __launch_bounds__(256) void k_attention(AttnLaunch a) {
    extern __shared__ float sm[];
    const int h = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int hd = a.head_dim, P = a.max_pos;
    const int QD = a.num_heads * hd;
    const int kvh = h / (a.num_heads / a.num_kv_heads);
    const int L = (a.d_pos ? *a.d_pos : a.pos_base) + i + 1;
    float* q = sm;
    float* red = sm + hd;
    float* sc = red + 8;
    for (int d = tid; d < hd; d += 256) q[d] = a.q[(size_t)i * QD + h * hd + d];
    __syncthreads();
    const float* K = a.k_cache + (size_t)kvh * P * hd;
    float lmax = -__builtin_huge_valf();
    for (int j = tid; j < L; j += 256) {
        float s = 0.0f;
        for (int d = 0; d < hd; d++) s = s + q[d] * K[(size_t)j * hd + d];
        s = s * a.scale;
        sc[j] = s;
        lmax = s > lmax ? s : lmax;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        float o = __shfl_xor(lmax, d, 64);
        lmax = o > lmax ? o : lmax;
    }
    if (lane == 0) red[wave] = lmax;
    __syncthreads();
    float mx = red[0];
    for (int w = 1; w < 4; w++) mx = red[w] > mx ? red[w] : mx;
    for (int j = tid; j < L; j += 256) sc[j] = expf_cr(sc[j] - mx);
    __syncthreads();
    if (wave == 0) {
        float acc = 0.0f;
        for (int j = lane; j < L; j += 64) acc = acc + sc[j];
        acc = wave_sum64(acc);
        if (lane == 0) red[4] = acc;
    }
    __syncthreads();
    const float sum = red[4];
    for (int j = tid; j < L; j += 256) sc[j] = __fdiv_rn(sc[j], sum);
    __syncthreads();
    const float* V = a.v_cache + (size_t)kvh * P * hd;
    for (int d = tid; d < hd; d += 256) {
        float o = 0.0f;
        for (int j = 0; j < L; j++) o = o + sc[j] * V[(size_t)j * hd + d];
        a.out[(size_t)i * QD + h * hd + d] = o;
    }
}


// ---- decode attention (one new position) ------------------------------------

// The q-head's query and, when this chunk holds the new position, the new
// key: RmsNorm per head then RoPE, computed by one wave (lane l holds
// elements l, l+64, ...).  Same arithmetic as k_qk_rope_kv.
__device__ __forceinline__ void norm_rope_head(const float* src, const float* w, const float* cs, const float* sn,
                                               int hd, float eps, float* dst) {
    const int lane = threadIdx.x & 63, R = hd / 2, per = hd / 64;
    float xb[8], y[8];
    float acc = 0.0f;
    for (int t = 0; t < per; t++) {
        float v = bf16_round(src[lane + 64 * t]);
        xb[t] = v;
        acc = acc + v * v;
    }
    acc = wave_sum64(acc);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)hd) + eps));
    for (int t = 0; t < per; t++) y[t] = bf16_round((xb[t] * inv) * bf16_round(w[lane + 64 * t]));
    for (int t = 0; t < per / 2; t++) {
        const int d = lane + 64 * t;
        const float c = cs[d & ~1], s = sn[d & ~1];
        const float x1 = y[t], x2 = y[t + per / 2];
        dst[d] = x1 * c - x2 * s;
        dst[d + R] = x2 * c + x1 * s;
    }
}

// grid (num_heads, max_pos / 64), block 64: scores of 64 positions of one
// q-head, s_j = (q . k_j sequential over head_dim) * scale.  The workgroup
// holding the new position also appends its key and value to the cache
// (the first q-head of each kv group writes; the others recompute the key).
__global__ __launch_bounds__(64) void k_attn_scores(AttnDecodeLaunch a) {
    __shared__ float qs[512];
    __shared__ float ks[512];
    const int h = blockIdx.x, c = blockIdx.y, lane = threadIdx.x;
    const int hd = a.head_dim, P = a.max_pos, groups = a.num_heads / a.num_kv_heads;
    const int kvh = h / groups;
    const int pos = a.d_pos ? *a.d_pos : a.pos_base;
    const int L = pos + 1;
    const int p = c * 64 + lane;
    if (c * 64 >= L) return;
    const int QD = a.num_heads * hd, KD = a.num_kv_heads * hd;
    const float* kc = a.k_cache + (size_t)kvh * P * hd;
    // key row of this lane's position (cached positions only), loaded first
    float4 kr[32];
    const bool cached = p < pos;
    if (cached) {
        const float4* src = (const float4*)(kc + (size_t)p * hd);
        for (int t = 0; t < hd / 4; t++) kr[t] = src[t];
    }
    const float* cs = a.cos_t + (size_t)pos * (hd / 2);
    const float* sn = a.sin_t + (size_t)pos * (hd / 2);
    norm_rope_head(a.qkv + h * hd, a.q_norm, cs, sn, hd, a.eps, qs);
    const bool has_new = pos >= c * 64 && pos < c * 64 + 64;
    if (has_new) {
        norm_rope_head(a.qkv + QD + kvh * hd, a.k_norm, cs, sn, hd, a.eps, ks);
        __syncthreads();
        if (h % groups == 0) {
            float* krow = a.k_cache + ((size_t)kvh * P + pos) * hd;
            float* vrow = a.v_cache + ((size_t)kvh * P + pos) * hd;
            const float* v = a.qkv + QD + KD + kvh * hd;
            for (int d = lane; d < hd; d += 64) {
                krow[d] = ks[d];
                vrow[d] = v[d];
            }
        }
    }
    __syncthreads();
    if (p >= L) return;
    float s = 0.0f;
    if (cached) {
        for (int t = 0; t < hd / 4; t++) {
            s = s + qs[4 * t] * kr[t].x;
            s = s + qs[4 * t + 1] * kr[t].y;
            s = s + qs[4 * t + 2] * kr[t].z;
            s = s + qs[4 * t + 3] * kr[t].w;
        }
    } else {
        for (int d = 0; d < hd; d++) s = s + qs[d] * ks[d];
    }
    a.scores[(size_t)h * P + p] = s * a.scale;
}

// grid (num_kv_heads), block 64 * groups * head_dim / 64: softmax of each
// q-head of the kv group (max, exp(s - max), SUM64, divide), then
// out[h][d] = sum_j p_j v_j[d] sequentially over j, V staged through LDS in
// chunks of 32 positions.
__global__ __launch_bounds__(1024) void k_attn_pv(AttnDecodeLaunch a) {
    extern __shared__ float sm[];
    const int kvh = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hd = a.head_dim, P = a.max_pos, groups = a.num_heads / a.num_kv_heads;
    const int L = (a.d_pos ? *a.d_pos : a.pos_base) + 1;
    const int nt = blockDim.x;
    float* pr = sm;                  // [groups][P] probabilities
    float* vt = pr + groups * P;     // [32][hd] staged values
    // softmax rows: wave w < groups handles q-head kvh*groups + w
    if (wave < groups) {
        const int h = kvh * groups + wave;
        const float* sc = a.scores + (size_t)h * P;
        float* p = pr + wave * P;
        float mx = -__builtin_huge_valf();
        for (int j = lane; j < L; j += 64) {
            float v = sc[j];
            p[j] = v;
            mx = v > mx ? v : mx;
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            float o = __shfl_xor(mx, d, 64);
            mx = o > mx ? o : mx;
        }
        float acc = 0.0f;
        for (int j = lane; j < L; j += 64) {
            float e = expf_cr(p[j] - mx);
            p[j] = e;
            acc = acc + e;
        }
        acc = wave_sum64(acc);
        for (int j = lane; j < L; j += 64) p[j] = __fdiv_rn(p[j], acc);
    }
    __syncthreads();
    const int hq = tid / hd, d = tid % hd;          // output element of this thread
    const float* V = a.v_cache + (size_t)kvh * P * hd;
    const float* p = pr + hq * P;
    float o = 0.0f;
    for (int j0 = 0; j0 < L; j0 += 32) {
        const int nj = min(32, L - j0);
        for (int i = tid * 4; i < nj * hd; i += nt * 4) *(float4*)(vt + i) = *(const float4*)(V + (size_t)j0 * hd + i);
        __syncthreads();
        if (hq < groups)
            for (int j = 0; j < nj; j++) o = o + p[j0 + j] * vt[j * hd + d];
        __syncthreads();
    }
    if (hq < groups) a.out[(size_t)(kvh * groups + hq) * hd + d] = o;
}

// RmsNorm of each row (src/rms_norm.rs:143-176), one wave per row.
__global__ __launch_bounds__(64) void k_rms_norm_rows(const float* __restrict__ x, const float* __restrict__ w, int dim,
                                                      float eps, float* __restrict__ y) {
    const int r = blockIdx.x, lane = threadIdx.x;
    const float* xr = x + (size_t)r * dim;
    float acc = 0.0f;
    for (int i = lane; i < dim; i += 64) {
        float v = bf16_round(xr[i]);
        acc = acc + v * v;
    }
    acc = wave_sum64(acc);
    const float mean = __fdiv_rn(acc, (float)dim);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(mean + eps));
    float* yr = y + (size_t)r * dim;
    for (int i = lane; i < dim; i += 64) yr[i] = bf16_round((bf16_round(xr[i]) * inv) * bf16_round(w[i]));
}

// act = silu(gate) * up (src/mlp.rs:151-164; silu src/tensor.rs:1978).
__global__ void k_silu_mul(const float* __restrict__ gu, int rows, int inter, float* __restrict__ act) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows * inter) return;
    size_t r = idx / inter, j = idx % inter;
    float g = gu[r * 2 * inter + j], u = gu[r * 2 * inter + inter + j];
    float s = __fdiv_rn(g, 1.0f + expf_cr(-g));
    act[idx] = s * u;
}

// Tensor::silu f32 branch (src/tensor.rs:1978): x / (1 + exp(-x)).
__global__ void k_silu(const float* __restrict__ x, size_t n, float* __restrict__ y) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    float v = x[idx];
    y[idx] = __fdiv_rn(v, 1.0f + expf_cr(-v));
}

// Greedy pick (src/generate.rs:153-174): maximum, last index on ties.
__global__ __launch_bounds__(1024) void k_argmax_step(const float* __restrict__ logits, int n, uint32_t* d_tok,
                                                      uint32_t* tokens_out, int* d_pos, int* d_step) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -__builtin_huge_valf();
    int bi = -1;
    for (int i = tid; i < n; i += 1024) {
        float v = logits[i];
        if (v > bv || v == bv) { bv = v; bi = i; }
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        float ov = __shfl_xor(bv, d, 64);
        int oi = __shfl_xor(bi, d, 64);
        if (ov > bv || (ov == bv && oi > bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++)
            if (sv[w] > bv || (sv[w] == bv && si[w] > bi)) { bv = sv[w]; bi = si[w]; }
        uint32_t tok = (uint32_t)(bi < 0 ? 0 : bi);
        *d_tok = tok;
        tokens_out[*d_step] = tok;
        *d_step = *d_step + 1;
        *d_pos = *d_pos + 1;
    }
}

inline unsigned grid1(size_t n, unsigned block) { return (unsigned)((n + block - 1) / block); }

}  // namespace

lq8_status launch_qk_rope_kv(hipStream_t s, const QkRopeLaunch& a) {
    if (a.head_dim % 128 || a.head_dim > 512)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "head_dim must be a multiple of 128 and at most 512");
    dim3 grid((unsigned)a.n, (unsigned)(a.num_heads + a.num_kv_heads));
    hipLaunchKernelGGL(k_qk_rope_kv, grid, dim3(64), 0, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_attention(hipStream_t s, const AttnLaunch& a) {
    size_t smem = ((size_t)a.head_dim + 8 + (size_t)a.max_pos) * sizeof(float);
    dim3 grid((unsigned)a.num_heads, (unsigned)a.n);
    hipLaunchKernelGGL(k_attention, grid, dim3(256), smem, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}


bool attention_decode_supported(int num_heads, int num_kv_heads, int head_dim, int max_pos) {
    const long long groups = num_heads / num_kv_heads;
    const long long lds = (groups * max_pos + 32ll * head_dim) * 4;
    return head_dim == 128 && groups * head_dim <= 1024 && lds <= 64 * 1024;
}

lq8_status launch_attention_decode(hipStream_t s, const AttnDecodeLaunch& a) {
    if (!attention_decode_supported(a.num_heads, a.num_kv_heads, a.head_dim, a.max_pos))
        return fail(LQ8_ERR_SHAPE_MISMATCH, "decode attention: unsupported head layout");
    const int groups = a.num_heads / a.num_kv_heads;
    hipLaunchKernelGGL(k_attn_scores, dim3((unsigned)a.num_heads, (unsigned)((a.max_pos + 63) / 64)), dim3(64), 0, s, a);
    LQ8_HIP(hipGetLastError());
    const int threads = ((groups * a.head_dim + 63) / 64) * 64;
    size_t smem = ((size_t)groups * a.max_pos + 32 * (size_t)a.head_dim) * sizeof(float);
    hipLaunchKernelGGL(k_attn_pv, dim3((unsigned)a.num_kv_heads), dim3(threads < 256 ? 256 : threads), smem, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_rms_norm_rows(hipStream_t s, const float* x, const float* w, int rows, int dim, float eps, float* y) {
    hipLaunchKernelGGL(k_rms_norm_rows, dim3((unsigned)rows), dim3(64), 0, s, x, w, dim, eps, y);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_silu_mul(hipStream_t s, const float* gu, int rows, int inter, float* act) {
    size_t n = (size_t)rows * inter;
    hipLaunchKernelGGL(k_silu_mul, dim3(grid1(n, 256)), dim3(256), 0, s, gu, rows, inter, act);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_silu(hipStream_t s, const float* x, size_t n, float* y) {
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_silu, dim3(grid1(n, 256)), dim3(256), 0, s, x, n, y);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_argmax_step(hipStream_t s, const float* logits, int n, uint32_t* d_tok, uint32_t* tokens_out,
                              int* d_pos, int* d_step) {
    hipLaunchKernelGGL(k_argmax_step, dim3(1), dim3(1024), 0, s, logits, n, d_tok, tokens_out, d_pos, d_step);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

}  // namespace lq8
