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
        // PV4 order: chunk c of 64 positions belongs to set c % 4; sets sum
        // their positions in order, then ((A0 + A1) + A2) + A3.
        float s4[4];
        for (int st = 0; st < 4; st++) {
            float o = 0.0f;
            for (int j0 = st * 64; j0 < L; j0 += 256) {
                const int je = min(j0 + 64, L);
                for (int j = j0; j < je; j++) o = o + sc[j] * V[(size_t)j * hd + d];
            }
            s4[st] = o;
        }
        a.out[(size_t)i * QD + h * hd + d] = ((s4[0] + s4[1]) + s4[2]) + s4[3];
    }
}


// ---- attention, one workgroup per (kv group, query) -------------------------

// RmsNorm per head then RoPE of one head vector held by one wave (lane l has
// elements l and l + 64), exactly as k_qk_rope_kv; src holds the projection
// as (base +) partials.
__device__ __forceinline__ void head_norm_rope(const float* src_p, int g_count, size_t stride, const float* w,
                                               const float* cs, const float* sn, float eps, float* dst) {
    const int lane = threadIdx.x & 63;
    float xb[2];
    float acc = 0.0f;
    for (int t = 0; t < 2; t++) {
        float s = 0.0f;
        for (int g = 0; g < g_count; g++) s = s + src_p[(size_t)g * stride + lane + 64 * t];
        float v = bf16_round(s);
        xb[t] = v;
        acc = acc + v * v;
    }
    acc = wave_sum64(acc);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, 128.0f) + eps));
    const float y0 = bf16_round((xb[0] * inv) * bf16_round(w[lane]));
    const float y1 = bf16_round((xb[1] * inv) * bf16_round(w[lane + 64]));
    const float c = cs[lane & ~1], s = sn[lane & ~1];
    dst[lane] = y0 * c - y1 * s;
    dst[lane + 64] = y1 * c + y0 * s;
}

// grid (num_kv_heads, n), block G * 512 (G = q-heads per kv head, head_dim 128).
// Decode (qkv_p set): the query heads and the new key come from the qkv
// projection partials; the new key and value are appended to the cache and
// used from LDS.  Prefill (q_rows set): normalized, rotated queries and a
// filled cache.  Then scores (q.k sequential over d, times scale), softmax
// (max, exp, SUM64, divide) and p.v in the PV4 order: thread group st of four
// accumulates the positions of chunks st, st + 4, ... in order, and the four
// partial sums are added in order.
__global__ __launch_bounds__(1024) void k_attn_group(AttnGroupLaunch a) {
    extern __shared__ float sm[];
    const int kvh = blockIdx.x, i = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.num_heads / a.num_kv_heads, T = G * 512, P = a.max_pos;
    const int QD = a.num_heads * 128, KD = a.num_kv_heads * 128;
    const int pos = (a.d_pos ? *a.d_pos : a.pos_base) + i;
    const int L = pos + 1;
    float* qs = sm;                  // [G][128]
    float* kn = qs + G * 128;        // [128] new key
    float* vn = kn + 128;            // [128] new value
    float* pr = vn + 128;            // [G][P] scores, then probabilities
    float* part = pr + G * P;        // [4][G * 128]
    const bool fused = a.qkv_p != nullptr;
    if (fused) {
        const float* cs = a.cos_t + (size_t)pos * 64;
        const float* sn = a.sin_t + (size_t)pos * 64;
        if (wave < G) {
            head_norm_rope(a.qkv_p + (kvh * G + wave) * 128, a.qkv_g, a.qkv_stride, a.q_norm, cs, sn, a.eps,
                           qs + wave * 128);
        } else if (wave == G) {
            head_norm_rope(a.qkv_p + QD + kvh * 128, a.qkv_g, a.qkv_stride, a.k_norm, cs, sn, a.eps, kn);
            float* krow = a.k_cache + ((size_t)kvh * P + pos) * 128;
            krow[lane] = kn[lane];
            krow[lane + 64] = kn[lane + 64];
        } else if (wave == G + 1) {
            float* vrow = a.v_cache + ((size_t)kvh * P + pos) * 128;
            for (int t = 0; t < 2; t++) {
                float s = 0.0f;
                for (int g = 0; g < a.qkv_g; g++) s = s + a.qkv_p[(size_t)g * a.qkv_stride + QD + KD + kvh * 128 + lane + 64 * t];
                vn[lane + 64 * t] = s;
                vrow[lane + 64 * t] = s;
            }
        }
    } else {
        for (int e = tid; e < G * 128; e += T) qs[e] = a.q_rows[(size_t)i * QD + kvh * G * 128 + e];
    }
    __syncthreads();
    // scores
    const float* K = a.k_cache + (size_t)kvh * P * 128;
    for (int j = tid; j < L; j += T) {
        float s[8];
        for (int h = 0; h < G; h++) s[h] = 0.0f;
        if (fused && j == pos) {
            for (int d = 0; d < 128; d++)
                for (int h = 0; h < G; h++) s[h] = s[h] + qs[h * 128 + d] * kn[d];
        } else {
            const float4* kr = (const float4*)(K + (size_t)j * 128);
            for (int t = 0; t < 32; t++) {
                const float4 k4 = kr[t];
                for (int h = 0; h < G; h++) {
                    const float* q = qs + h * 128 + 4 * t;
                    s[h] = s[h] + q[0] * k4.x;
                    s[h] = s[h] + q[1] * k4.y;
                    s[h] = s[h] + q[2] * k4.z;
                    s[h] = s[h] + q[3] * k4.w;
                }
            }
        }
        for (int h = 0; h < G; h++) pr[h * P + j] = s[h] * a.scale;
    }
    __syncthreads();
    // softmax per q-head, one wave each
    if (wave < G) {
        float* p = pr + wave * P;
        float mx = -__builtin_huge_valf();
        for (int j = lane; j < L; j += 64) mx = p[j] > mx ? p[j] : mx;
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
    // p.v, PV4 order
    {
        const int st = tid / (G * 128), r = tid % (G * 128), hq = r / 128, d = r % 128;
        const float* V = a.v_cache + (size_t)kvh * P * 128;
        const float* p = pr + hq * P;
        float o = 0.0f;
        for (int j0 = st * 64; j0 < L; j0 += 256) {
            const int je = min(j0 + 64, L);
            for (int j = j0; j < je; j++) {
                const float v = (fused && j == pos) ? vn[d] : V[(size_t)j * 128 + d];
                o = o + p[j] * v;
            }
        }
        part[st * G * 128 + r] = o;
    }
    __syncthreads();
    for (int r = tid; r < G * 128; r += T) {
        const float o = ((part[r] + part[G * 128 + r]) + part[2 * G * 128 + r]) + part[3 * G * 128 + r];
        a.out[(size_t)i * QD + kvh * G * 128 + r] = o;
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


bool attention_group_supported(int num_heads, int num_kv_heads, int head_dim, int max_pos) {
    if (head_dim != 128 || num_heads % num_kv_heads) return false;
    const long long G = num_heads / num_kv_heads;
    const long long lds = (G * 128 + 256 + G * max_pos + 4 * G * 128) * 4;
    return G >= 1 && G <= 2 && lds <= 64 * 1024;
}

lq8_status launch_attention_group(hipStream_t s, const AttnGroupLaunch& a) {
    if (!attention_group_supported(a.num_heads, a.num_kv_heads, 128, a.max_pos))
        return fail(LQ8_ERR_SHAPE_MISMATCH, "grouped attention: unsupported head layout");
    const int G = a.num_heads / a.num_kv_heads;
    size_t smem = ((size_t)G * 128 + 256 + (size_t)G * a.max_pos + 4 * (size_t)G * 128) * sizeof(float);
    hipLaunchKernelGGL(k_attn_group, dim3((unsigned)a.num_kv_heads, (unsigned)a.n), dim3(G * 512), smem, s, a);
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
