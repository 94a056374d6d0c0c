// gemv.hip -- decode-time Q8_0 GEMV (W8A32) for gfx950.
//
// A weight is stored as 64-row tiles; each tile row is cut into groups of 8
// Q8_0 blocks (256 values, 16 KiB of codes per tile).  One wave owns one
// (tile, group): lane r streams row r's codes with two coalesced 1 KiB loads
// per block, keeps them in registers, and accumulates
//   p_b = fmaf chain over the block's 32 codes,   a_g = fmaf(p_b, d_b, a_g).
// The row result is y = ((0 + a_0) + a_1) + ... in group order.
//
// Two output modes:
//   FINAL     one workgroup per tile, one wave per group; the group partials
//             meet in LDS and wave 0 writes y (plus an optional residual).
//   PARTIALS  one single-wave workgroup per (tile, group), so even a
//             1024-row weight occupies the whole chip; the partials a_g are
//             written out and the consuming kernel adds them in group order
//             while it stages its own input (no extra launch, no
//             cross-workgroup synchronisation).
// Inputs may themselves arrive as partials: x_i = base_i + S_i with
// S_i = ((0 + P_0,i) + P_1,i) + ...  (the residual add of the reference,
// base + projection, with the projection completed first).
//
// Every workgroup issues its weight loads before it stages the input, so the
// HBM latency of the weights overlaps the staging.
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

enum OutMode : int { OUT_FINAL = 0, OUT_PARTIALS = 1 };

__device__ __forceinline__ float dot16(u32x4 v, const float* __restrict__ x, float p) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 xv = *(const float4*)(x + 4 * i);
        p = fmaf((float)(int8_t)(w[i] & 0xFF), xv.x, p);
        p = fmaf((float)(int8_t)((w[i] >> 8) & 0xFF), xv.y, p);
        p = fmaf((float)(int8_t)((w[i] >> 16) & 0xFF), xv.z, p);
        p = fmaf((float)(int8_t)(w[i] >> 24), xv.w, p);
    }
    return p;
}

// Input element i: base_i + (partials summed in group order).
__device__ __forceinline__ float load_x(const GemvLaunch& a, int i) {
    if (a.xg == 0) return a.x[i];
    float s = 0.0f;
    for (int g = 0; g < a.xg; g++) s = s + a.xp[(size_t)g * a.xstride + i];
    return a.x ? a.x[i] + s : s;
}

// Stage the input range [k0, k1) (relative to k0) into LDS.
template <int XS, int NT>
__device__ __forceinline__ void stage_range(const GemvLaunch& a, int k0, int k1, float* xs, float* red) {
    const int tid = threadIdx.x;
    if (XS == XS_PLAIN) {
        if (a.xg == 0) {
            for (int i = k0 + tid * 4; i < k1; i += NT * 4) *(float4*)(xs + i - k0) = *(const float4*)(a.x + i);
        } else {
            for (int i = k0 + tid; i < k1; i += NT) xs[i - k0] = load_x(a, i);
        }
    } else if (XS == XS_SILU) {
        // silu(gate) * up (src/mlp.rs:151-164; silu src/tensor.rs:1978)
        for (int i = k0 + tid; i < k1; i += NT) {
            float g = load_x(a, i), u = load_x(a, a.k + i);
            xs[i - k0] = __fdiv_rn(g, 1.0f + expf_cr(-g)) * u;
        }
    } else {
        // RmsNorm (src/rms_norm.rs:143-176) of the whole input with the SUM64
        // order; workgroup 0 also stores the (pre-norm) input when asked.
        if (tid < 64) {
            float acc = 0.0f;
            for (int i = tid; i < a.k; i += 64) {
                float xv = load_x(a, i);
                if (a.x_out && blockIdx.x == 0) a.x_out[i] = xv;
                float v = bf16_round(xv);
                acc = acc + v * v;
            }
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) acc = acc + __shfl_xor(acc, d, 64);
            if (tid == 0) red[0] = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)a.k) + a.eps));
        }
        __syncthreads();
        const float inv = red[0];
        for (int i = k0 + tid; i < k1; i += NT)
            xs[i - k0] = bf16_round((bf16_round(load_x(a, i)) * inv) * bf16_round(a.norm_w[i]));
    }
}

// W waves per workgroup.  FINAL: workgroup = tile, wave = group (W >= groups).
// PARTIALS: W == 1, workgroup = (tile, group) with tile = blockIdx / groups.
template <int XS, int W, int MODE>
__global__ __launch_bounds__(64 * W) void k_gemv2(GemvLaunch a) {
    extern __shared__ float smem[];
    float* xs = smem;  // staged input range
    const int nb = a.k / 32;
    const int ngroups = (nb + GROUP_BLOCKS - 1) / GROUP_BLOCKS;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    size_t tile;
    int g;
    if (MODE == OUT_PARTIALS) {
        tile = blockIdx.x / ngroups;
        g = blockIdx.x % ngroups;
    } else {
        tile = blockIdx.x;
        g = wave;
    }
    const int range = MODE == OUT_PARTIALS ? GROUP_BLOCKS * 32 : a.k;
    float* red = xs + range;  // 4 floats
    float* part = red + 4;    // W * 64 floats
    const int b0 = g * GROUP_BLOCKS;
    const int nblk = g < ngroups ? min(GROUP_BLOCKS, nb - b0) : 0;
    const int k0 = MODE == OUT_PARTIALS ? b0 * 32 : 0;
    const int k1 = MODE == OUT_PARTIALS ? min(a.k, k0 + GROUP_BLOCKS * 32) : a.k;

    const int8_t* cb = a.codes + (tile * nb + b0) * 2048 + lane * 16;
    const uint16_t* sb = a.scales + (tile * nb + b0) * 64 + lane;
    float acc = 0.0f;
    if (nblk == GROUP_BLOCKS) {
        // weights first: 8 blocks x 2 x 16 bytes per lane, plus the scales
        u32x4 lo[GROUP_BLOCKS], hi[GROUP_BLOCKS];
        uint16_t ds[GROUP_BLOCKS];
#pragma unroll
        for (int i = 0; i < GROUP_BLOCKS; i++) {
            lo[i] = __builtin_nontemporal_load((const u32x4*)(cb + i * 2048));
            hi[i] = __builtin_nontemporal_load((const u32x4*)(cb + i * 2048 + 1024));
            ds[i] = sb[i * 64];
        }
        stage_range<XS, 64 * W>(a, k0, k1, xs, red);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < GROUP_BLOCKS; i++) {
            const float* xb = xs + (b0 + i) * 32 - k0;
            float p = dot16(lo[i], xb, 0.0f);
            p = dot16(hi[i], xb + 16, p);
            acc = fmaf(p, f16_bits_to_f32(ds[i]), acc);
        }
    } else {
        // tail group (fewer than 8 blocks) or an idle wave
        stage_range<XS, 64 * W>(a, k0, k1, xs, red);
        __syncthreads();
        for (int i = 0; i < nblk; i++) {
            u32x4 l = *(const u32x4*)(cb + i * 2048);
            u32x4 h = *(const u32x4*)(cb + i * 2048 + 1024);
            const float* xb = xs + (b0 + i) * 32 - k0;
            float p = dot16(l, xb, 0.0f);
            p = dot16(h, xb + 16, p);
            acc = fmaf(p, f16_bits_to_f32(sb[i * 64]), acc);
        }
    }
    if (MODE == OUT_PARTIALS) {
        const size_t tiles = (size_t)(a.n + TILE_ROWS - 1) / TILE_ROWS;
        a.partials[(size_t)g * tiles * TILE_ROWS + tile * TILE_ROWS + lane] = acc;
    } else {
        part[wave * 64 + lane] = acc;
        __syncthreads();
        if (wave == 0) {
            float y = 0.0f;
            for (int gg = 0; gg < ngroups; gg++) y = y + part[gg * 64 + lane];
            const size_t row = tile * TILE_ROWS + lane;
            if (row < (size_t)a.n) {
                if (a.resid) y = a.resid[row] + y;
                a.y[row] = y;
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_combine(const float* __restrict__ base, const float* __restrict__ partials,
                                                 int groups, size_t stride, int n, float* __restrict__ y) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = 0.0f;
    for (int g = 0; g < groups; g++) s = s + partials[(size_t)g * stride + i];
    y[i] = base ? base[i] + s : s;
}

template <int XS, int W, int MODE>
lq8_status launch_v2(hipStream_t s, const GemvLaunch& a, unsigned grid) {
    const int range = MODE == OUT_PARTIALS ? GROUP_BLOCKS * 32 : a.k;
    size_t smem = (size_t)(range + 4 + W * 64) * sizeof(float);
    hipLaunchKernelGGL((k_gemv2<XS, W, MODE>), dim3(grid), dim3(64 * W), smem, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

template <int XS>
lq8_status dispatch(hipStream_t s, const GemvLaunch& a) {
    const int nb = a.k / 32, ngroups = (nb + GROUP_BLOCKS - 1) / GROUP_BLOCKS;
    const size_t tiles = (a.n + TILE_ROWS - 1) / TILE_ROWS;
    if (a.partials) {
        if (tiles * TILE_ROWS * (size_t)ngroups > (size_t)a.partials_cap)
            return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: partial buffer too small");
        return launch_v2<XS, 1, OUT_PARTIALS>(s, a, (unsigned)(tiles * ngroups));
    }
    if (a.k > 8192) return launch_gemv_tile_wg(s, (XSource)XS, a);
    const unsigned grid = (unsigned)tiles;
    if (ngroups <= 4) return launch_v2<XS, 4, OUT_FINAL>(s, a, grid);
    if (ngroups <= 8) return launch_v2<XS, 8, OUT_FINAL>(s, a, grid);
    if (ngroups <= 16) return launch_v2<XS, 16, OUT_FINAL>(s, a, grid);
    return launch_gemv_tile_wg(s, (XSource)XS, a);
}

}  // namespace

lq8_status launch_gemv(hipStream_t s, XSource xs, const GemvLaunch& a) {
    if (a.k <= 0 || a.k % 32 || a.n <= 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k must be a positive multiple of 32");
    if (a.k > 16384) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k > 16384 not supported");
    switch (xs) {
        case XS_PLAIN: return dispatch<XS_PLAIN>(s, a);
        case XS_RMSNORM: return dispatch<XS_RMSNORM>(s, a);
        default: return dispatch<XS_SILU>(s, a);
    }
}

lq8_status launch_combine(hipStream_t s, const float* base, const float* partials, int groups, size_t stride, int n,
                          float* y) {
    if (n <= 0) return LQ8_OK;
    hipLaunchKernelGGL(k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, base, partials, groups, stride, n,
                       y);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

size_t gemv_partial_stride(int n) { return (size_t)((n + TILE_ROWS - 1) / TILE_ROWS) * TILE_ROWS; }
int gemv_groups(int k) { return (k / 32 + GROUP_BLOCKS - 1) / GROUP_BLOCKS; }

}  // namespace lq8
