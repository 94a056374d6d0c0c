// gemv.hip -- decode-time Q8_0 GEMV (W8A32) for gfx950.
//
// Work split.  A weight is stored as 64-row tiles; each tile row is cut into
// groups of 8 Q8_0 blocks (256 values, 16 KiB of codes per tile).  One wave
// owns one (tile, group): lane r streams row r's codes with two coalesced
// 1 KiB loads per block, keeps them in registers, and accumulates
//   p_b = fmaf chain over the block's 32 codes,  a_g = fmaf(p_b, d_b, a_g).
// The group partials of a tile are then added in group order,
//   y = ((0 + a_0) + a_1) + ...,
// either inside the workgroup (all groups of the tile in one workgroup) or,
// when the groups are spread over several workgroups to occupy the chip,
// by the last workgroup of the tile to finish (a device-scope counter decides
// which one; it sums the partials in group order, so the result does not
// depend on the finishing order).  Every workgroup issues its weight loads
// before it stages the input vector, so the HBM latency of the weights
// overlaps the staging.
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

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

// Stage x[k0, k1) (relative to k0) into LDS for the given x-source.
template <int XS, int NT>
__device__ __forceinline__ void stage_range(const GemvLaunch& a, int k0, int k1, float* xs, float* red) {
    const int tid = threadIdx.x;
    if (XS == XS_PLAIN) {
        for (int i = k0 + tid * 4; i < k1; i += NT * 4) *(float4*)(xs + i - k0) = *(const float4*)(a.x + i);
    } else if (XS == XS_SILU) {
        // silu(gate) * up (src/mlp.rs:151-164; silu src/tensor.rs:1978)
        for (int i = k0 + tid; i < k1; i += NT) {
            float g = a.x[i], u = a.x[a.k + i];
            xs[i - k0] = __fdiv_rn(g, 1.0f + expf_cr(-g)) * u;
        }
    } else {
        // RmsNorm (src/rms_norm.rs:143-176) over the whole vector with the
        // SUM64 order, then the normalized values of this range.
        if (tid < 64) {
            float acc = 0.0f;
            for (int i = tid; i < a.k; i += 64) {
                float v = bf16_round(a.x[i]);
                acc = acc + v * v;
            }
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) acc = acc + __shfl_xor(acc, d, 64);
            if (tid == 0) red[0] = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)a.k) + a.eps));
        }
        __syncthreads();
        const float inv = red[0];
        for (int i = k0 + tid; i < k1; i += NT)
            xs[i - k0] = bf16_round((bf16_round(a.x[i]) * inv) * bf16_round(a.norm_w[i]));
    }
}

__device__ __forceinline__ void store_row(const GemvLaunch& a, size_t row, float acc) {
    if (row < (size_t)a.n) {
        if (a.resid) acc = a.resid[row] + acc;
        a.y[row] = acc;
    }
}

// W waves per workgroup; workgroup `blockIdx.x` covers tile blockIdx.x / wpt
// and groups [gs*W, gs*W + W) with gs = blockIdx.x % wpt.
template <int XS, int W, bool SPLIT>
__global__ __launch_bounds__(64 * W) void k_gemv2(GemvLaunch a) {
    extern __shared__ float smem[];
    float* xs = smem;                 // W * 256 floats
    float* red = xs + W * 256;        // 4 floats
    float* part = red + 4;            // W * 64 floats
    int* flag = (int*)(part + W * 64);
    const int nb = a.k / 32;
    const int ngroups = (nb + GROUP_BLOCKS - 1) / GROUP_BLOCKS;
    const int wpt = (ngroups + W - 1) / W;
    const size_t tile = blockIdx.x / wpt;
    const int gs = blockIdx.x % wpt;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = gs * W + wave;
    const int b0 = g * GROUP_BLOCKS;
    const int nblk = g < ngroups ? min(GROUP_BLOCKS, nb - b0) : 0;

    // 1) weights first: 8 blocks x 2 x 16 bytes per lane, plus scales
    const int8_t* cb = a.codes + (tile * nb + b0) * 2048 + lane * 16;
    const uint16_t* sb = a.scales + (tile * nb + b0) * 64 + lane;
    const int k0 = gs * W * GROUP_BLOCKS * 32;
    const int k1 = min(a.k, k0 + W * GROUP_BLOCKS * 32);
    float acc = 0.0f;
    if (nblk == GROUP_BLOCKS) {
        u32x4 lo[GROUP_BLOCKS], hi[GROUP_BLOCKS];
        uint16_t ds[GROUP_BLOCKS];
#pragma unroll
        for (int i = 0; i < GROUP_BLOCKS; i++) {
            lo[i] = __builtin_nontemporal_load((const u32x4*)(cb + i * 2048));
            hi[i] = __builtin_nontemporal_load((const u32x4*)(cb + i * 2048 + 1024));
            ds[i] = sb[i * 64];
        }
        // 2) the input range this workgroup needs
        stage_range<XS, 64 * W>(a, k0, k1, xs, red);
        __syncthreads();
        // 3) the group partial
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
    // 4) groups of the tile, in order
    if (!SPLIT) {
        part[wave * 64 + lane] = acc;
        __syncthreads();
        if (wave == 0) {
            float y = 0.0f;
            for (int gg = 0; gg < ngroups; gg++) y = y + part[gg * 64 + lane];
            store_row(a, tile * TILE_ROWS + lane, y);
        }
    } else {
        if (g < ngroups) a.partials[(tile * ngroups + g) * 64 + lane] = acc;
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0) *flag = atomicAdd(&a.counters[tile], 1) == wpt - 1;
        __syncthreads();
        if (*flag) {
            __threadfence();
            if (wave == 0) {
                const float* pp = a.partials + tile * ngroups * 64 + lane;
                float y = 0.0f;
                for (int gg = 0; gg < ngroups; gg++) y = y + __builtin_nontemporal_load(pp + gg * 64);
                store_row(a, tile * TILE_ROWS + lane, y);
            }
            if (threadIdx.x == 0) a.counters[tile] = 0;
        }
    }
}

template <int XS, int W, bool SPLIT>
lq8_status launch_v2(hipStream_t s, const GemvLaunch& a, unsigned grid) {
    size_t smem = (size_t)(W * 256 + 4 + W * 64 + 4) * sizeof(float);
    hipLaunchKernelGGL((k_gemv2<XS, W, SPLIT>), dim3(grid), dim3(64 * W), smem, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

template <int XS>
lq8_status dispatch(hipStream_t s, const GemvLaunch& a) {
    const int nb = a.k / 32, ngroups = (nb + GROUP_BLOCKS - 1) / GROUP_BLOCKS;
    const size_t tiles = (a.n + TILE_ROWS - 1) / TILE_ROWS;
    // Large outputs fill the chip with 4-wave workgroups; small ones spread
    // their groups over one-wave workgroups and combine through the counters.
    const int W = tiles >= 256 ? 4 : 1;
    const int wpt = (ngroups + W - 1) / W;
    const bool split = wpt > 1;
    if (split && (!a.partials || !a.counters || tiles > (size_t)a.counters_cap ||
                  tiles * (size_t)ngroups * 64 > (size_t)a.partials_cap))
        return launch_gemv_tile_wg(s, (XSource)XS, a);
    const unsigned grid = (unsigned)(tiles * wpt);
    if (W == 4) return split ? launch_v2<XS, 4, true>(s, a, grid) : launch_v2<XS, 4, false>(s, a, grid);
    return split ? launch_v2<XS, 1, true>(s, a, grid) : launch_v2<XS, 1, false>(s, a, grid);
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

}  // namespace lq8
