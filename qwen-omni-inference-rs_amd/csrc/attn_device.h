// attn_device.h -- decode attention building blocks shared by the segment
// attention kernels (model_kernels.hip) and the persistent decode kernel
// (decode_persistent.hip): per-head RmsNorm + RoPE, the segment's scores,
// softmax partials and P.V chain, in the orders the CPU oracle restates
// (SUM64 denominators, q.k sequential over head_dim, P.V sequential over
// positions).  Workgroups of NT threads (ATT_THREADS unless stated).
// PIN_TID: the thread index is taken through tid_here() (for callers inside
// long-lived loops, where hoisted index math would stay live throughout).
#pragma once

#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

constexpr int SEG = ATT_SEG;

template <bool PIN>
__device__ __forceinline__ int thread_x() {
    return PIN ? tid_here() : (int)threadIdx.x;
}
// LDS row stride of staged keys: rows start on 16-byte boundaries (b128 reads
// and writes) and consecutive rows 4 banks apart (conflict-free per 8 lanes)
constexpr int KPAD = 132;

// LDS float offsets of the staged K/V rows (16-byte aligned for float4 stores)
__host__ __device__ inline int seg_ks_off(int G) { return (G * 128 + 256 + G * SEG + 2 * G + 3) & ~3; }
__host__ __device__ inline int rows_ks_off(int G) { return (G * 128 + G * SEG + 6 * G + 3) & ~3; }

// max fold in the SUM64 pattern: a = (o > a ? o : a) with o the value of lane
// l ^ d, d = 32, 16, 8, 4, 2, 1.
template <int D>
__device__ __forceinline__ float max_step(float a) {
    const float o = lane_xor<D>(a);
    return o > a ? o : a;
}
__device__ __forceinline__ float wave_max64(float a) {
    a = max_step<32>(a);
    a = max_step<16>(a);
    a = max_step<8>(a);
    a = max_step<4>(a);
    a = max_step<2>(a);
    a = max_step<1>(a);
    return a;
}

// RmsNorm of one head vector (src/attention.rs:350-358 with src/rms_norm.rs:143-176)
// then RoPE (src/rope.rs:270-297) at table row cs/sn; one wave, lane l has
// elements l and l + 64 (head_dim 128).
// c, s: the table entries of the lane's rotation pair (cs[lane & ~1], sn[lane & ~1]).
__device__ __forceinline__ void head_norm_rope_cs(float s0, float s1, float w0, float w1, float c, float s, float eps,
                                                  float* dst) {
    const int lane = threadIdx.x & 63;
    const float x0 = bf16_round(s0), x1 = bf16_round(s1);
    float acc = 0.0f;
    acc = acc + x0 * x0;
    acc = acc + x1 * x1;
    acc = wave_sum64(acc);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, 128.0f) + eps));
    const float y0 = bf16_round((x0 * inv) * bf16_round(w0));
    const float y1 = bf16_round((x1 * inv) * bf16_round(w1));
    dst[lane] = y0 * c - y1 * s;
    dst[lane + 64] = y1 * c + y0 * s;
}
__device__ __forceinline__ void head_norm_rope_vals(float s0, float s1, float w0, float w1, const float* cs,
                                                    const float* sn, float eps, float* dst) {
    const int lane = threadIdx.x & 63;
    head_norm_rope_cs(s0, s1, w0, w1, cs[lane & ~1], sn[lane & ~1], eps, dst);
}
__device__ __forceinline__ void head_norm_rope(const float* src, const float* w, const float* cs, const float* sn,
                                               float eps, float* dst) {
    const int lane = threadIdx.x & 63;
    // all loads first, then the arithmetic
    const float s0 = src[lane], s1 = src[lane + 64];
    const float w0 = w[lane], w1 = w[lane + 64];
    head_norm_rope_vals(s0, s1, w0, w1, cs, sn, eps, dst);
}

// Shared per-segment work of the attention kernels (blocks of NT threads).
// Stages the keys of positions [js, js + nj) into ks (row `knew_row` of the
// segment, if >= 0, from knew), computes the scores of the G query heads in
// qs into sc[h][j], then per head m_c, e_j (into sc) and l_c (mlc[2h], mlc[2h+1]).
// kreg/vreg: this thread's prefetched float4s (ATT_SEG * 32 / NT) of the segment's K and V rows.
// The loads are unconditional (rows past the segment read row js instead) so
// they are all in flight together; the values of those rows, and of the new
// position's row (written by this kernel), are never used.
template <int NT = ATT_THREADS, bool PIN_TID = false>
__device__ __forceinline__ void seg_load(const float* __restrict__ Kc, const float* __restrict__ Vc, int js, int nj,
                                         float4* kreg, float4* vreg) {
    const int tid = thread_x<PIN_TID>();
#pragma unroll
    for (int u = 0; u < ATT_SEG * 32 / NT; u++) {
        const int f = tid + u * NT;  // float4 index in the [64][32] segment
        const int j = f >> 5, c4 = f & 31;
        const size_t row = (size_t)js + (j < nj ? j : 0);
        kreg[u] = *(const float4*)(Kc + row * 128 + c4 * 4);
        vreg[u] = *(const float4*)(Vc + row * 128 + c4 * 4);
    }
}

// The same loads before the position is known: rows js .. js + 63 clamped to
// the cache capacity (rows past the position are loaded and never used).
template <int NT = ATT_THREADS, bool PIN_TID = false>
__device__ __forceinline__ void seg_load_capacity(const float* __restrict__ Kc, const float* __restrict__ Vc, int js,
                                                  int max_pos, float4* kreg, float4* vreg) {
    const int tid = thread_x<PIN_TID>();
#pragma unroll
    for (int u = 0; u < ATT_SEG * 32 / NT; u++) {
        const int f = tid + u * NT;
        const int j = f >> 5, c4 = f & 31;
        const size_t row = (size_t)min(js + j, max_pos - 1);
        kreg[u] = *(const float4*)(Kc + row * 128 + c4 * 4);
        vreg[u] = *(const float4*)(Vc + row * 128 + c4 * 4);
    }
}

// q . k over head_dim 128, sequential over d from +0 (s = s + q[d] * k[d]);
// q and k 16-byte aligned in LDS, read 4 elements at a time.
__device__ __forceinline__ float qk_dot128(const float* q, const float* k) {
    const float4* q4 = (const float4*)q;
    const float4* k4 = (const float4*)k;
    float s = 0.0f;
#pragma unroll
    for (int d4 = 0; d4 < 32; d4++) {
        const float4 a = q4[d4], b = k4[d4];
        s = s + a.x * b.x;
        s = s + a.y * b.y;
        s = s + a.z * b.z;
        s = s + a.w * b.w;
    }
    return s;
}

// LDS_SYNC: the barriers order LDS only (lds_sync: the caller's own global
// stores are not waited for), for callers that keep global visibility apart.
template <int NT = ATT_THREADS, bool PIN_TID = false, bool LDS_SYNC = false>
__device__ __forceinline__ void seg_scores(const float4* kreg, int nj, int knew_row, const float* knew, const float* qs,
                                           int G, float scale, float* ks, float* sc, float* mlc) {
    const int tid = thread_x<PIN_TID>(), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll
    for (int u = 0; u < ATT_SEG * 32 / NT; u++) {
        const int f = tid + u * NT;
        const int j = f >> 5, c4 = f & 31;
        if (j < nj) {
            float4 v = kreg[u];
            if (j == knew_row) v = *(const float4*)(knew + c4 * 4);
            *(float4*)(ks + j * KPAD + c4 * 4) = v;
        }
    }
    if (LDS_SYNC) lds_sync();
    else __syncthreads();
    for (int t = tid; t < G * SEG; t += NT) {
        const int h = t / SEG, j = t % SEG;
        if (j < nj) sc[h * SEG + j] = qk_dot128(qs + h * 128, ks + j * KPAD) * scale;
    }
    if (LDS_SYNC) lds_sync();
    else __syncthreads();
    for (int h = wave; h < G; h += NT / 64) {
        const float s = lane < nj ? sc[h * SEG + lane] : -__builtin_huge_valf();
        const float mc = wave_max64(s);
        const float e = lane < nj ? expf_cr(s - mc) : 0.0f;
        const float lc = wave_sum64(e);
        if (lane < nj) sc[h * SEG + lane] = e;
        if (lane == 0) {
            mlc[2 * h] = mc;
            mlc[2 * h + 1] = lc;
        }
    }
}

// o = sum_j e[j] * vs[j][d] for j = 0 .. nj - 1 in order, from +0.  Sixteen
// steps per batch: their LDS reads go out together (e is 16-byte aligned and
// wave-uniform), then the chain; the order of the adds is unchanged.
__device__ __forceinline__ float pv_chain(const float* e, const float* vs, int d, int nj) {
    float o = 0.0f;
    int j = 0;
    for (; j + 16 <= nj; j += 16) {
        float4 ev[4];
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) ev[q] = *(const float4*)(e + j + 4 * q);
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = vs[(j + u) * 128 + d];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            o = o + ev[q].x * v[4 * q];
            o = o + ev[q].y * v[4 * q + 1];
            o = o + ev[q].z * v[4 * q + 2];
            o = o + ev[q].w * v[4 * q + 3];
        }
    }
    for (; j < nj; j++) o = o + e[j] * vs[j * 128 + d];
    return o;
}

// V rows of the segment into vs [64][128] (row vnew_row from vnew).
template <int NT = ATT_THREADS, bool PIN_TID = false>
__device__ __forceinline__ void seg_stage_v(const float4* vreg, int nj, int vnew_row, const float* vnew, float* vs) {
    const int tid = thread_x<PIN_TID>();
#pragma unroll
    for (int u = 0; u < ATT_SEG * 32 / NT; u++) {
        const int f = tid + u * NT;
        const int j = f >> 5, c4 = f & 31;
        if (j < nj) {
            float4 v = vreg[u];
            if (j == vnew_row) v = *(const float4*)(vnew + c4 * 4);
            *(float4*)(vs + j * 128 + c4 * 4) = v;
        }
    }
}

}  // namespace lq8
