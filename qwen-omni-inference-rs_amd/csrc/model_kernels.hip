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
            float* kt = a.k_cache_t + (size_t)kvh * hd * a.max_pos;
            kt[(size_t)d * a.max_pos + pos] = o1;
            kt[(size_t)(d + R) * a.max_pos + pos] = o2;
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
    const float* KT = a.k_cache_t + (size_t)kvh * hd * P;
    float lmax = -__builtin_huge_valf();
    for (int j = tid; j < L; j += 256) {
        float s = 0.0f;
        for (int d = 0; d < hd; d++) s = s + q[d] * KT[(size_t)d * P + j];
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
