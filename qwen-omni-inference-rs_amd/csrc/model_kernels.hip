// model_kernels.hip -- decoder kernels around the Q8_0 linears (gfx950).
//
// Orders follow the CPU oracle exactly:
//   SUM64   lane l (of one 64-lane wave) accumulates elements l, l+64, ... from
//           0; the partials fold at distances 32, 16, 8, 4, 2, 1.  Used for the
//           RMSNorm sum of squares and the softmax denominator.
//   scores  q.k sequential over head_dim (src/tensor.rs:2846-2915), then
//           times 1/sqrt(head_dim).
//   ATTN    positions in segments of 64: per segment m_c = max s, e = exp(s - m_c),
//           l_c = SUM64(e), o_c = sum_j e_j v_j (j in order); then the running
//           (m, num, den) update m' = max(m, m_c), a = exp(m - m'),
//           b = exp(m_c - m'), num = num a + b o_c, den = den a + b l_c; the
//           output is num / den.
#include "attn_device.h"
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

// q/k RmsNorm per head, RoPE and KV-cache append for n rows (prefill).
// grid (n, num_heads + num_kv_heads), block 64.
__global__ __launch_bounds__(64) void k_qk_rope_kv(QkRopeLaunch a) {
    const int i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int QD = a.num_heads * 128, KD = a.num_kv_heads * 128, row = QD + 2 * KD;
    const int pos = (a.d_pos ? *a.d_pos : a.pos_base) + i;
    const bool isq = h < a.num_heads;
    const float* src = a.qkv + (size_t)i * row + (isq ? h * 128 : QD + (h - a.num_heads) * 128);
    const float* cs = a.cos_t + (size_t)pos * 64;
    const float* sn = a.sin_t + (size_t)pos * 64;
    if (isq) {
        head_norm_rope(src, a.q_norm, cs, sn, a.eps, a.q_out + (size_t)i * QD + h * 128);
    } else {
        const int kvh = h - a.num_heads;
        head_norm_rope(src, a.k_norm, cs, sn, a.eps, a.k_cache + ((size_t)kvh * a.max_pos + pos) * 128);
        const float* v = a.qkv + (size_t)i * row + QD + KD + kvh * 128;
        float* vc = a.v_cache + ((size_t)kvh * a.max_pos + pos) * 128;
        vc[lane] = v[lane];
        vc[lane + 64] = v[lane + 64];
    }
}


// Decode attention, one workgroup per (kv head, group of HG of its G query
// heads, segment slot y), which takes the segments of 64 positions y, y +
// gridDim.y, ... in use (ROUNDS; otherwise there are as many slots as
// segments of capacity, and the instance without the loop keeps its
// registers: 73 VGPRs against 148).  Every workgroup normalizes and rotates its HG query
// heads; the workgroups of the last segment also normalize and rotate the
// new key and use key and value from LDS, and the one of head group 0
// appends them to the cache at the position.  Output: per (segment, q head)
// o_c[128], m_c, l_c at part[(c * H + h) * ATT_PART_STRIDE].
template <bool ROUNDS>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_seg(AttnSegLaunch a) {
    extern __shared__ float sm[];
    const int G = a.num_heads / a.num_kv_heads, HG = a.head_group, NG = G / HG;
    const int kvh = blockIdx.x / NG, hg = blockIdx.x - kvh * NG, c0 = blockIdx.y, b = blockIdx.z;
    const int h0 = kvh * G + hg * HG;  // this workgroup's first query head
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int QD = a.num_heads * 128, KD = a.num_kv_heads * 128;
    a.qkv += b * a.qkv_stride;
    a.k_cache += b * a.kv_stride;
    a.v_cache += b * a.kv_stride;
    a.part += b * a.part_stride;
    const float* Kc = a.k_cache + (size_t)kvh * a.max_pos * 128;
    const float* Vc = a.v_cache + (size_t)kvh * a.max_pos * 128;
    // Loads that do not depend on the position go out before it arrives: the
    // K/V rows of the first ATT_EARLY_SEGS segments of a single sequence
    // (almost always in use; later segments, and batches, whose idle
    // workgroups would multiply the waste, wait) and this wave's first head
    // vector (q head `wave`, or the new k / v).
    float4 kreg[ATT_F4], vreg[ATT_F4];
    const bool early = c0 < ATT_EARLY_SEGS && gridDim.z == 1;
    if (early) seg_load_capacity(Kc, Vc, c0 * SEG, a.max_pos, kreg, vreg);
    float x0 = 0.0f, x1 = 0.0f, n0 = 0.0f, n1 = 0.0f;
    if (wave < HG + 2) {
        const float* src = wave < HG ? a.qkv + (h0 + wave) * 128
                                     : a.qkv + QD + (wave == HG ? 0 : KD) + kvh * 128;
        x0 = src[lane];
        x1 = src[lane + 64];
        if (wave <= HG) {
            const float* w = wave < HG ? a.q_norm : a.k_norm;
            n0 = w[lane];
            n1 = w[lane + 64];
        }
    }
    const int pos = a.d_pos ? a.d_pos[b] : a.pos_base;
    const int L = pos + 1;
    const int C = (L + SEG - 1) / SEG;
    // before any barrier: the whole workgroup leaves (a position outside the
    // cache writes nothing)
    if (c0 >= C || pos < 0 || pos >= a.max_pos) return;
    float* qs = sm;                      // [HG][128]
    float* kn = qs + HG * 128;           // [128]
    float* vn = kn + 128;                // [128]
    float* sc = vn + 128;                // [HG][64]
    float* mlc = sc + HG * SEG;          // [HG][2]
    float* ks = sm + seg_ks_off(HG);     // [64][KPAD], later vs [64][128]
    const float* cs = a.cos_t + (size_t)pos * 64;
    const float* sn = a.sin_t + (size_t)pos * 64;
    // segments c0, c0 + gridDim.y, ... (every workgroup of the launch takes
    // the same number of rounds of its own; the rounds after the first wait
    // for the previous one's reads of the LDS regions)
    for (int c = c0;;) {
        const int js = c * SEG;
        const int nj = min(SEG, L - js);
        const bool last = c == C - 1;
        const int newrow = last ? pos - js : -1;
        if (!(early && c == c0)) seg_load(Kc, Vc, js, nj, kreg, vreg);
        for (int t = wave; t < HG + 2; t += ATT_THREADS / 64) {
            if (t < HG) {
                if (t == wave) head_norm_rope_vals(x0, x1, n0, n1, cs, sn, a.eps, qs + t * 128);
                else head_norm_rope(a.qkv + (h0 + t) * 128, a.q_norm, cs, sn, a.eps, qs + t * 128);
            } else if (t == HG && last) {
                if (t == wave) head_norm_rope_vals(x0, x1, n0, n1, cs, sn, a.eps, kn);
                else head_norm_rope(a.qkv + QD + kvh * 128, a.k_norm, cs, sn, a.eps, kn);
                if (hg == 0) {
                    float* kr = a.k_cache + ((size_t)kvh * a.max_pos + pos) * 128;
                    kr[lane] = kn[lane];
                    kr[lane + 64] = kn[lane + 64];
                }
            } else if (t == HG + 1 && last) {
                const float* v = a.qkv + QD + KD + kvh * 128;
                const float v0 = t == wave ? x0 : v[lane], v1 = t == wave ? x1 : v[lane + 64];
                vn[lane] = v0;
                vn[lane + 64] = v1;
                if (hg == 0) {
                    float* vr = a.v_cache + ((size_t)kvh * a.max_pos + pos) * 128;
                    vr[lane] = v0;
                    vr[lane + 64] = v1;
                }
            }
        }
        __syncthreads();
        seg_scores(kreg, nj, newrow, kn, qs, HG, a.scale, ks, sc, mlc);
        __syncthreads();
        seg_stage_v(vreg, nj, newrow, vn, ks);
        __syncthreads();
        for (int t = tid; t < HG * 128; t += ATT_THREADS) {
            const int h = t >> 7, d = t & 127;
            const float o = pv_chain(sc + h * SEG, ks, d, nj);
            float* p = a.part + ((size_t)c * a.num_heads + h0 + h) * ATT_PART_STRIDE;
            p[d] = o;
            if (d == 0) {
                p[128] = mlc[2 * h];
                p[129] = mlc[2 * h + 1];
            }
        }
        if (!ROUNDS) break;
        c += gridDim.y;
        if (c >= C) break;
        __syncthreads();  // the next round's writes wait for this round's reads of the LDS regions
    }
}

// Attention output of one sequence's head from its per-segment partials,
// one thread per head dimension d: the running update over the segments in
// order, m' = max(m, m_c), a = exp(m - m'), b = exp(m_c - m'),
// num = num * a + b * o_c, den = den * a + b * l_c; out = num / den (the
// arithmetic of the o-projection's XS_ATTN staging, thread by thread).
__global__ __launch_bounds__(128) void k_attn_combine(const float* __restrict__ part, size_t part_stride,
                                                      const int* __restrict__ d_pos, int H, int cmax,
                                                      float* __restrict__ out) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const int C = min(max(d_pos[b], 0) / SEG + 1, cmax);
    const float* pb = part + b * part_stride;
    float m = -__builtin_huge_valf(), den = 0.0f, num = 0.0f;
    for (int c = 0; c < C; c++) {
        const float* p = pb + ((size_t)c * H + h) * ATT_PART_STRIDE;
        const float mc = p[128], lc = p[129];
        const float mn = m > mc ? m : mc;
        const float ea = expf_cr(m - mn), eb = expf_cr(mc - mn);
        den = den * ea + eb * lc;
        num = num * ea + eb * p[d];
        m = mn;
    }
    out[(size_t)b * H * 128 + h * 128 + d] = __fdiv_rn(num, den);
}

// Attention over n query rows with a filled cache (prefill): one workgroup
// per (kv head, R consecutive rows), R * G <= 16.  The segments run in order
// with the running update; each K/V segment is staged once for the R rows,
// and a row whose positions end before a segment skips it (its arithmetic is
// the single-row sequence exactly).
template <int R>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_rows(AttnRowsLaunch a) {
    extern __shared__ float sm[];
    const int kvh = blockIdx.x, i0 = blockIdx.y * R;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = a.num_heads / a.num_kv_heads, RG = R * G;
    const int QD = a.num_heads * 128;
    const int nr = min(R, a.n - i0);
    const int Lmax = a.pos_base + i0 + nr;  // positions of the workgroup's last row
    const float* Kc = a.k_cache + (size_t)kvh * a.max_pos * 128;
    const float* Vc = a.v_cache + (size_t)kvh * a.max_pos * 128;
    float* qs = sm;                      // [R][G][128]
    float* sc = qs + RG * 128;           // [R][G][64]
    float* mlc = sc + RG * SEG;          // [R][G][2]
    float* run = mlc + 2 * RG;           // [R][G][4]: m, den, a, b
    float* ks = sm + rows_ks_off(RG);    // [64][KPAD], later vs [64][128]
    for (int e = tid; e < RG * 128; e += ATT_THREADS) {
        const int rr = e / (G * 128), w = e - rr * G * 128;
        qs[e] = a.q_rows[(size_t)(i0 + min(rr, nr - 1)) * QD + kvh * G * 128 + w];
    }
    for (int h = tid; h < RG; h += ATT_THREADS) {
        run[4 * h] = -__builtin_huge_valf();
        run[4 * h + 1] = 0.0f;
    }
    // thread t < R * G * 128 (looping) keeps num for (row, head, d) = (t / (G * 128), (t / 128) % G, t % 128)
    constexpr int MAXR = 16 * 128 / ATT_THREADS;
    float num[MAXR];
#pragma unroll
    for (int r = 0; r < MAXR; r++) num[r] = 0.0f;
    float4 kreg[ATT_F4], vreg[ATT_F4];
    for (int js = 0; js < Lmax; js += SEG) {
        const int njmax = min(SEG, Lmax - js);
        seg_load(Kc, Vc, js, njmax, kreg, vreg);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < ATT_F4; u++) {
            const int f = tid + u * ATT_THREADS;
            const int j = f >> 5, c4 = f & 31;
            if (j < njmax) {
                *(float4*)(ks + j * KPAD + c4 * 4) = kreg[u];
            }
        }
        __syncthreads();
        // scores q.k, sequential over d, then times the scale (one thread per (row, head, position))
        for (int t = tid; t < RG * SEG; t += ATT_THREADS) {
            const int rh = t / SEG, j = t - rh * SEG, rr = rh / G;
            const int nj = min(SEG, a.pos_base + i0 + rr + 1 - js);
            if (rr < nr && j < nj) sc[rh * SEG + j] = qk_dot128(qs + rh * 128, ks + j * KPAD) * a.scale;
        }
        __syncthreads();
        // segment softmax per (row, head): max, exp, SUM64 denominator
        for (int rh = wave; rh < RG; rh += ATT_THREADS / 64) {
            const int rr = rh / G;
            const int nj = min(SEG, a.pos_base + i0 + rr + 1 - js);
            if (rr < nr && nj > 0) {
                const float sv = lane < nj ? sc[rh * SEG + lane] : -__builtin_huge_valf();
                const float mc = wave_max64(sv);
                const float e = lane < nj ? expf_cr(sv - mc) : 0.0f;
                const float lc = wave_sum64(e);
                if (lane < nj) sc[rh * SEG + lane] = e;
                if (lane == 0) {
                    mlc[2 * rh] = mc;
                    mlc[2 * rh + 1] = lc;
                }
            }
        }
        __syncthreads();
        for (int rh = tid; rh < RG; rh += ATT_THREADS) {
            const int rr = rh / G;
            if (rr < nr && a.pos_base + i0 + rr + 1 - js > 0) {
                const float m = run[4 * rh], mc = mlc[2 * rh];
                const float mn = m > mc ? m : mc;
                const float ea = expf_cr(m - mn), eb = expf_cr(mc - mn);
                run[4 * rh] = mn;
                run[4 * rh + 1] = run[4 * rh + 1] * ea + eb * mlc[2 * rh + 1];
                run[4 * rh + 2] = ea;
                run[4 * rh + 3] = eb;
            }
        }
        seg_stage_v(vreg, njmax, -1, nullptr, ks);
        __syncthreads();
#pragma unroll
        for (int r = 0; r < MAXR; r++) {
            const int t = tid + r * ATT_THREADS;
            if (t < RG * 128) {
                const int rh = t >> 7, d = t & 127, rr = rh / G;
                const int nj = min(SEG, a.pos_base + i0 + rr + 1 - js);
                if (rr < nr && nj > 0) {
                    const float o = pv_chain(sc + rh * SEG, ks, d, nj);
                    num[r] = num[r] * run[4 * rh + 2] + run[4 * rh + 3] * o;
                }
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < MAXR; r++) {
        const int t = tid + r * ATT_THREADS;
        if (t < RG * 128) {
            const int rh = t >> 7, d = t & 127, rr = rh / G, h = rh - rr * G;
            if (rr < nr)
                a.out[(size_t)(i0 + rr) * QD + (kvh * G + h) * 128 + d] = __fdiv_rn(num[r], run[4 * rh + 1]);
        }
    }
}

// RmsNorm of each row (src/rms_norm.rs:143-176), one wave per row.
template <int U>
__global__ __launch_bounds__(64) void k_rms_norm_rows(const float* __restrict__ x, const float* __restrict__ w, int dim,
                                                      float eps, float* __restrict__ y) {
    // U <= 32: the row and the norm weights stay in registers (loaded together);
    // U == 0: longer rows, two passes of 16 loads in flight per lane.
    const int r = blockIdx.x, lane = threadIdx.x;
    const float* xr = x + (size_t)r * dim;
    float* yr = y + (size_t)r * dim;
    if (U > 0) {
        constexpr int UU = U > 0 ? U : 1;
        float v[UU], wn[UU];
#pragma unroll
        for (int u = 0; u < UU; u++) {
            v[u] = xr[min(lane + 64 * u, dim - 1)];
            wn[u] = w[min(lane + 64 * u, dim - 1)];
        }
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < UU; u++)
            if (lane + 64 * u < dim) {
                const float b = bf16_round(v[u]);
                acc = acc + b * b;
            }
        acc = wave_sum64(acc);
        const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)dim) + eps));
#pragma unroll
        for (int u = 0; u < UU; u++)
            if (lane + 64 * u < dim) yr[lane + 64 * u] = bf16_round((bf16_round(v[u]) * inv) * bf16_round(wn[u]));
        return;
    }
    constexpr int L = 16;  // loads in flight per lane
    float acc = 0.0f;
    for (int i0 = lane; i0 < dim; i0 += 64 * L) {
        float v[L];
#pragma unroll
        for (int u = 0; u < L; u++) v[u] = xr[min(i0 + 64 * u, dim - 1)];
#pragma unroll
        for (int u = 0; u < L; u++)
            if (i0 + 64 * u < dim) {
                const float b = bf16_round(v[u]);
                acc = acc + b * b;
            }
    }
    acc = wave_sum64(acc);
    const float mean = __fdiv_rn(acc, (float)dim);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(mean + eps));
    for (int i0 = lane; i0 < dim; i0 += 64 * L) {
        float v[L], wv[L];
#pragma unroll
        for (int u = 0; u < L; u++) {
            const int i = min(i0 + 64 * u, dim - 1);
            v[u] = xr[i];
            wv[u] = w[i];
        }
#pragma unroll
        for (int u = 0; u < L; u++)
            if (i0 + 64 * u < dim) yr[i0 + 64 * u] = bf16_round((bf16_round(v[u]) * inv) * bf16_round(wv[u]));
    }
}

// act = silu(gate) * up (src/mlp.rs:151-164; silu src/tensor.rs:1978).
__global__ void k_silu_mul(const float* __restrict__ gu, int rows, int inter, float* __restrict__ act) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows * inter) return;
    const size_t r = idx / inter, j = idx % inter;
    const float g = gu[r * 2 * inter + j], u = gu[r * 2 * inter + inter + j];
    const float s = __fdiv_rn(g, 1.0f + expf_cr(-g));
    act[idx] = s * u;
}

// Tensor::silu f32 branch (src/tensor.rs:1978): x / (1 + exp(-x)).
__global__ void k_silu(const float* __restrict__ x, size_t n, float* __restrict__ y) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const float v = x[idx];
    y[idx] = __fdiv_rn(v, 1.0f + expf_cr(-v));
}

inline unsigned grid1(size_t n, unsigned block) { return (unsigned)((n + block - 1) / block); }

constexpr int ATT_WG_TARGET = 512;  // decode attention workgroups sought per launch (2 per CU)
constexpr int ATT_MIN_SLOTS = 8;    // segment slots at least (512 positions without a second round)

size_t seg_smem(int G) { return ((size_t)seg_ks_off(G) + (size_t)SEG * KPAD) * sizeof(float); }
size_t rows_smem(int G) { return ((size_t)rows_ks_off(G) + (size_t)SEG * KPAD) * sizeof(float); }

}  // namespace

bool attention_supported(int num_heads, int num_kv_heads, int head_dim) {
    return head_dim == 128 && num_kv_heads > 0 && num_heads % num_kv_heads == 0 &&
           num_heads / num_kv_heads <= ATT_MAX_GROUP;
}

lq8_status launch_qk_rope_kv(hipStream_t s, const QkRopeLaunch& a) {
    if (a.head_dim != 128) return fail(LQ8_ERR_SHAPE_MISMATCH, "head_dim must be 128");
    const dim3 grid((unsigned)a.n, (unsigned)(a.num_heads + a.num_kv_heads));
    hipLaunchKernelGGL(k_qk_rope_kv, grid, dim3(64), 0, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_attention_seg(hipStream_t s, const AttnSegLaunch& a) {
    if (!attention_supported(a.num_heads, a.num_kv_heads, 128))
        return fail(LQ8_ERR_SHAPE_MISMATCH, "attention: unsupported head layout");
    const int G = a.num_heads / a.num_kv_heads;
    const int cmax = (a.max_pos + SEG - 1) / SEG;
    if (a.batch <= 0) return fail(LQ8_ERR_INVALID_ARG, "attention: batch must be positive");
    AttnSegLaunch b = a;
    if (b.head_group <= 0 || G % b.head_group) b.head_group = G;
    const int NG = G / b.head_group;
    // segment slots: all cmax segments up to about ATT_WG_TARGET workgroups
    // (at least ATT_MIN_SLOTS slots); a long max_positions (Qwen3's 40960:
    // 640 segments) no longer launches a workgroup per segment of capacity,
    // almost all of them idle, and a workgroup loops over its segments
    const int per_slot = a.num_kv_heads * NG * a.batch;
    const int slots = std::min(cmax, std::max(ATT_MIN_SLOTS, (ATT_WG_TARGET + per_slot - 1) / per_slot));
    const dim3 grid((unsigned)(a.num_kv_heads * NG), (unsigned)slots, (unsigned)a.batch);
    if (slots < cmax) hipLaunchKernelGGL(k_attn_seg<true>, grid, dim3(ATT_THREADS), seg_smem(b.head_group), s, b);
    else hipLaunchKernelGGL(k_attn_seg<false>, grid, dim3(ATT_THREADS), seg_smem(b.head_group), s, b);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_attention_combine(hipStream_t s, const float* part, size_t part_stride, const int* d_pos,
                                    int batch, int num_heads, int cmax, float* out) {
    if (batch <= 0 || num_heads <= 0 || cmax <= 0) return LQ8_OK;
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)num_heads, (unsigned)batch), dim3(128), 0, s, part, part_stride,
                       d_pos, num_heads, cmax, out);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_attention_rows(hipStream_t s, const AttnRowsLaunch& a) {
    if (!attention_supported(a.num_heads, a.num_kv_heads, 128))
        return fail(LQ8_ERR_SHAPE_MISMATCH, "attention: unsupported head layout");
    const int G = a.num_heads / a.num_kv_heads;
    // rows per workgroup: R * G <= 16 (the per-thread output registers)
    const int R = G <= 4 ? 4 : G <= 8 ? 2 : 1;
    const dim3 grid((unsigned)a.num_kv_heads, (unsigned)((a.n + R - 1) / R));
    if (R == 4) hipLaunchKernelGGL(k_attn_rows<4>, grid, dim3(ATT_THREADS), rows_smem(R * G), s, a);
    else if (R == 2) hipLaunchKernelGGL(k_attn_rows<2>, grid, dim3(ATT_THREADS), rows_smem(R * G), s, a);
    else hipLaunchKernelGGL(k_attn_rows<1>, grid, dim3(ATT_THREADS), rows_smem(R * G), s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_rms_norm_rows(hipStream_t s, const float* x, const float* w, int rows, int dim, float eps, float* y) {
    const dim3 grid((unsigned)rows);
    const int u = (dim + 63) / 64;
    if (u <= 4) hipLaunchKernelGGL(k_rms_norm_rows<4>, grid, dim3(64), 0, s, x, w, dim, eps, y);
    else if (u <= 8) hipLaunchKernelGGL(k_rms_norm_rows<8>, grid, dim3(64), 0, s, x, w, dim, eps, y);
    else if (u <= 16) hipLaunchKernelGGL(k_rms_norm_rows<16>, grid, dim3(64), 0, s, x, w, dim, eps, y);
    else if (u <= 32) hipLaunchKernelGGL(k_rms_norm_rows<32>, grid, dim3(64), 0, s, x, w, dim, eps, y);
    else hipLaunchKernelGGL(k_rms_norm_rows<0>, grid, dim3(64), 0, s, x, w, dim, eps, y);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_silu_mul(hipStream_t s, const float* gu, int rows, int inter, float* act) {
    const size_t n = (size_t)rows * inter;
    if (!n) return LQ8_OK;
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

}  // namespace lq8
