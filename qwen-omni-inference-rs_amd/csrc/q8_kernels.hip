// q8_kernels.hip -- Q8_0 format, GEMV (W8A32) and GEMM (W8A8 int8 MFMA) for gfx950.
//
// Accumulation orders (identical to the CPU oracle, so results are bitwise
// equal):
//   GEMV  row n: p_b = fmaf chain over the 32 codes of block b (j = 0..31,
//         from 0); a_g = fmaf(p_b, d_b, a_g) over the (up to) 8 blocks of
//         group g, from 0; y = y + a_g over groups, from 0.
//   GEMM  (m, n): I_b exact int32 from one v_mfma_i32_32x32x32_i8;
//         s_b = dw_b * dx_b; a_g = fmaf((float)I_b, s_b, a_g) over the group;
//         y = y + a_g over groups.
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

constexpr int WG = 256;

__device__ __forceinline__ size_t code_off(size_t tile, size_t nb, size_t b, int half, int r) {
    return ((tile * nb + b) * 2 + half) * 1024 + (size_t)r * 16;
}

__device__ __forceinline__ size_t scale_off(size_t tile, size_t nb, size_t b, int r) {
    return (tile * nb + b) * 64 + r;
}

// Store one quantized block of row `row` into the tiled layout.
__device__ __forceinline__ void store_tiled(int8_t* codes, size_t nb, size_t row, size_t b, const int* q) {
    size_t tile = row / TILE_ROWS;
    int r = (int)(row % TILE_ROWS);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        w[i] = (uint32_t)(q[4 * i] & 0xFF) | ((uint32_t)(q[4 * i + 1] & 0xFF) << 8) |
               ((uint32_t)(q[4 * i + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * i + 3] & 0xFF) << 24);
    uint4 lo = make_uint4(w[0], w[1], w[2], w[3]);
    uint4 hi = make_uint4(w[4], w[5], w[6], w[7]);
    *(uint4*)(codes + code_off(tile, nb, b, 0, r)) = lo;
    *(uint4*)(codes + code_off(tile, nb, b, 1, r)) = hi;
}

__device__ __forceinline__ void quantize32(const float* x, int* q, QBlock* qb) {
    float amax = block_amax(x);
    *qb = block_scale(amax);
    float id = block_inv(qb->d);
#pragma unroll
    for (int j = 0; j < 32; j++) q[j] = quant_code(x[j], id);
}

// ---- format kernels --------------------------------------------------------

__global__ void k_quantize_weight_f32(const float* __restrict__ src, size_t n_rows, size_t row0, size_t nb,
                                      int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    size_t r = idx / nb, b = idx % nb;
    float x[32];
    const float4* s4 = (const float4*)(src + r * nb * 32 + b * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 v = s4[i];
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
    int q[32];
    QBlock qb;
    quantize32(x, q, &qb);
    size_t row = row0 + r;
    store_tiled(codes, nb, row, b, q);
    scales[scale_off(row / TILE_ROWS, nb, b, (int)(row % TILE_ROWS))] = qb.d16;
}

__global__ void k_quantize_aos(const float* __restrict__ src, size_t nblocks, uint8_t* __restrict__ dst) {
    size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    float x[32];
#pragma unroll
    for (int j = 0; j < 32; j++) x[j] = src[b * 32 + j];
    int q[32];
    QBlock qb;
    quantize32(x, q, &qb);
    uint8_t* o = dst + b * BLOCK_BYTES;
    o[0] = (uint8_t)(qb.d16 & 0xFF);
    o[1] = (uint8_t)(qb.d16 >> 8);
#pragma unroll
    for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(q[j] & 0xFF);
}

__global__ void k_repack_aos(const uint8_t* __restrict__ aos, size_t n_rows, size_t nb, size_t row0,
                             int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    size_t r = idx / nb, b = idx % nb;
    const uint8_t* blk = aos + idx * BLOCK_BYTES;
    int q[32];
#pragma unroll
    for (int j = 0; j < 32; j++) q[j] = (int)(int8_t)blk[2 + j];
    size_t row = row0 + r;
    store_tiled(codes, nb, row, b, q);
    scales[scale_off(row / TILE_ROWS, nb, b, (int)(row % TILE_ROWS))] = (uint16_t)(blk[0] | (blk[1] << 8));
}

__global__ void k_unpack_aos(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales, size_t row0,
                             size_t n_rows, size_t nb, uint8_t* __restrict__ aos) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    size_t row = row0 + idx / nb, b = idx % nb;
    size_t tile = row / TILE_ROWS;
    int r = (int)(row % TILE_ROWS);
    uint8_t* o = aos + idx * BLOCK_BYTES;
    uint16_t d = scales[scale_off(tile, nb, b, r)];
    o[0] = (uint8_t)(d & 0xFF);
    o[1] = (uint8_t)(d >> 8);
    const int8_t* lo = codes + code_off(tile, nb, b, 0, r);
    const int8_t* hi = codes + code_off(tile, nb, b, 1, r);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        o[2 + j] = (uint8_t)lo[j];
        o[18 + j] = (uint8_t)hi[j];
    }
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// N(0, std) from a counter-based generator: each element pair (2i, 2i+1) of
// the tensor's row-major order takes one SplitMix64 hash of (seed, stream, i)
// through Box-Muller.
__global__ void k_random_weight(size_t n_rows, size_t row0, size_t nb, uint64_t key, float stddev,
                                int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    size_t r = idx / nb, b = idx % nb;
    size_t row = row0 + r;
    float x[32];
    size_t pair0 = (r * nb * 32 + b * 32) / 2;
#pragma unroll 4
    for (int i = 0; i < 16; i++) {
        uint64_t h = splitmix64(key + (pair0 + i) * 0xD1B54A32D192ED03ull);
        float u1 = ((float)(uint32_t)(h >> 40) + 1.0f) * 5.9604644775390625e-8f;
        float u2 = (float)(uint32_t)((h >> 16) & 0xFFFFFFu) * 5.9604644775390625e-8f;
        float rad = sqrtf(-2.0f * logf(u1));
        float th = 6.283185307179586f * u2;
        x[2 * i] = stddev * rad * cosf(th);
        x[2 * i + 1] = stddev * rad * sinf(th);
    }
    int q[32];
    QBlock qb;
    quantize32(x, q, &qb);
    store_tiled(codes, nb, row, b, q);
    scales[scale_off(row / TILE_ROWS, nb, b, (int)(row % TILE_ROWS))] = qb.d16;
}

// y[i, c] = d * q for rows ids[i] (or row0 + i when ids is null): exact.
__global__ void k_dequant_rows(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales, size_t nb,
                               const uint32_t* __restrict__ ids, size_t row0, size_t nrows, float* __restrict__ y) {
    size_t k = nb * 32;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nrows * k) return;
    size_t i = idx / k, c = idx % k;
    size_t row = ids ? (size_t)ids[i] : row0 + i;
    size_t tile = row / TILE_ROWS, b = c / 32;
    int r = (int)(row % TILE_ROWS), j = (int)(c % 32);
    float d = f16_bits_to_f32(scales[scale_off(tile, nb, b, r)]);
    int8_t q = codes[code_off(tile, nb, b, j >> 4, r) + (j & 15)];
    y[idx] = d * (float)q;
}

// ---- activation quantization (tiled A operand of the GEMM) ----------------

__global__ void k_quantize_act(const float* __restrict__ x, int m, int k, int8_t* __restrict__ codes,
                               float* __restrict__ scales32) {
    size_t nb = (size_t)k / 32;
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)m * nb) return;
    size_t r = idx / nb, b = idx % nb;
    float v[32];
    const float4* s4 = (const float4*)(x + r * (size_t)k + b * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        float4 t = s4[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    int q[32];
    QBlock qb;
    quantize32(v, q, &qb);
    store_tiled(codes, nb, r, b, q);
    scales32[scale_off(r / TILE_ROWS, nb, b, (int)(r % TILE_ROWS))] = f16_bits_to_f32(qb.d16);
}

// ---- GEMV ------------------------------------------------------------------

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// p = fmaf chain over the 16 codes in v against x[0..15], in order.
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

// Stage the GEMV input vector into LDS according to the x-source.
template <int XS>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, const float* __restrict__ norm_w, float eps,
                                        int k, float* xs, float* red) {
    const int tid = threadIdx.x;
    if (XS == XS_PLAIN) {
        for (int i = tid * 4; i < k; i += WG * 4) *(float4*)(xs + i) = *(const float4*)(x + i);
    } else if (XS == XS_SILU) {
        for (int i = tid; i < k; i += WG) {
            float g = x[i], u = x[k + i];
            float s = __fdiv_rn(g, 1.0f + expf_cr(-g));
            xs[i] = s * u;
        }
    } else {
        // RMSNorm (src/rms_norm.rs:143-176) with the SUM64 order: lane l sums
        // bf16(x_i)^2 for i = l, l+64, ...; the 64 partials fold at distances
        // 32, 16, 8, 4, 2, 1.
        if (tid < 64) {
            float a = 0.0f;
            for (int i = tid; i < k; i += 64) {
                float v = bf16_round(x[i]);
                a = a + v * v;
            }
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) a = a + __shfl_xor(a, d, 64);
            if (tid == 0) {
                float mean = __fdiv_rn(a, (float)k);
                red[0] = __fdiv_rn(1.0f, __builtin_sqrtf(mean + eps));
            }
        }
        __syncthreads();
        float inv = red[0];
        for (int i = tid; i < k; i += WG) {
            float v = bf16_round(x[i]);
            xs[i] = bf16_round((v * inv) * bf16_round(norm_w[i]));
        }
    }
}

// One 64-row tile: 4 waves split the groups, partials meet in LDS.
__device__ __forceinline__ void gemv_tile(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
                                          int nb, size_t tile, const float* xs, float* part, int n, float* __restrict__ y,
                                          const float* __restrict__ resid) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ngroups = (nb + GROUP_BLOCKS - 1) / GROUP_BLOCKS;
    const int8_t* cb = codes + tile * (size_t)nb * 2048 + (size_t)lane * 16;
    const uint16_t* sb = scales + tile * (size_t)nb * 64 + lane;
    for (int g = wave; g < ngroups; g += WG / 64) {
        const int b0 = g * GROUP_BLOCKS;
        const int nblk = min(GROUP_BLOCKS, nb - b0);
        float acc = 0.0f;
        if (nblk == GROUP_BLOCKS) {
            u32x4 lo[GROUP_BLOCKS], hi[GROUP_BLOCKS];
            uint16_t ds[GROUP_BLOCKS];
#pragma unroll
            for (int i = 0; i < GROUP_BLOCKS; i++) {
                const int8_t* p = cb + (size_t)(b0 + i) * 2048;
                lo[i] = __builtin_nontemporal_load((const u32x4*)p);
                hi[i] = __builtin_nontemporal_load((const u32x4*)(p + 1024));
                ds[i] = sb[(size_t)(b0 + i) * 64];
            }
#pragma unroll
            for (int i = 0; i < GROUP_BLOCKS; i++) {
                const float* xb = xs + (b0 + i) * 32;
                float p = dot16(lo[i], xb, 0.0f);
                p = dot16(hi[i], xb + 16, p);
                acc = fmaf(p, f16_bits_to_f32(ds[i]), acc);
            }
        } else {
            for (int i = 0; i < nblk; i++) {
                const int8_t* p = cb + (size_t)(b0 + i) * 2048;
                u32x4 l = *(const u32x4*)p;
                u32x4 h = *(const u32x4*)(p + 1024);
                const float* xb = xs + (b0 + i) * 32;
                float pp = dot16(l, xb, 0.0f);
                pp = dot16(h, xb + 16, pp);
                acc = fmaf(pp, f16_bits_to_f32(sb[(size_t)(b0 + i) * 64]), acc);
            }
        }
        part[g * 64 + lane] = acc;
    }
    __syncthreads();
    if (wave == 0) {
        float acc = 0.0f;
        for (int g = 0; g < ngroups; g++) acc = acc + part[g * 64 + lane];
        size_t row = tile * TILE_ROWS + lane;
        if (row < (size_t)n) {
            if (resid) acc = resid[row] + acc;
            y[row] = acc;
        }
    }
}

template <int XS>
__global__ __launch_bounds__(WG) void k_gemv(GemvLaunch a) {
    extern __shared__ float smem[];
    float* xs = smem;
    float* red = smem + a.k;
    float* part = red + 4;
    stage_x<XS>(a.x, a.norm_w, a.eps, a.k, xs, red);
    __syncthreads();
    gemv_tile(a.codes, a.scales, a.k / 32, blockIdx.x, xs, part, a.n, a.y, a.resid);
}

__global__ __launch_bounds__(WG) void k_gemv_grouped(const GemvProblemDev* __restrict__ probs, int count) {
    extern __shared__ float smem[];
    // find the problem owning this tile (tile_begin is ascending)
    int lo = 0, hi = count - 1;
    const int t = blockIdx.x;
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (probs[mid].tile_begin <= t) lo = mid;
        else hi = mid - 1;
    }
    const GemvProblemDev p = probs[lo];
    float* xs = smem;
    float* part = smem + p.k + 4;
    stage_x<XS_PLAIN>(p.x, nullptr, 0.0f, p.k, xs, nullptr);
    __syncthreads();
    gemv_tile(p.codes, p.scales, p.k / 32, (size_t)(t - p.tile_begin), xs, part, p.n, p.y, nullptr);
}

// ---- GEMM (W8A8, v_mfma_i32_32x32x32_i8) -------------------------------------

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Workgroup tile 64 (m) x 64 (n); wave w owns the 32x32 sub-tile (w>>1, w&1).
// Accumulator layout of the 32x32 MFMA: lane l holds column l%32, register r
// holds row 8*(r/4) + 4*(l/32) + r%4.
__global__ __launch_bounds__(WG) void k_gemm(const int8_t* __restrict__ xq, const float* __restrict__ xs32, int m,
                                             const int8_t* __restrict__ wc, const uint16_t* __restrict__ ws, int n,
                                             int nb, float* __restrict__ y, const float* __restrict__ resid, int ldy,
                                             int col0) {
    const int nt = blockIdx.x, mt = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, r32 = lane & 31;
    const int8_t* ab = xq + (size_t)mt * nb * 2048 + half * 1024 + (wm * 32 + r32) * 16;
    const int8_t* bb = wc + (size_t)nt * nb * 2048 + half * 1024 + (wn * 32 + r32) * 16;
    const float* dxb = xs32 + (size_t)mt * nb * 64 + wm * 32 + 4 * half;
    const uint16_t* dwb = ws + (size_t)nt * nb * 64 + wn * 32 + r32;
    float yacc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) yacc[r] = 0.0f;
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int b0 = 0; b0 < nb; b0 += GROUP_BLOCKS) {
        const int b1 = min(b0 + GROUP_BLOCKS, nb);
        float acc[16];
#pragma unroll
        for (int r = 0; r < 16; r++) acc[r] = 0.0f;
        for (int b = b0; b < b1; b++) {
            v4i av = *(const v4i*)(ab + (size_t)b * 2048);
            v4i bv = *(const v4i*)(bb + (size_t)b * 2048);
            v16i isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zero, 0, 0, 0);
            const float dw = f16_bits_to_f32(dwb[(size_t)b * 64]);
            const float* dx = dxb + (size_t)b * 64;
            float4 d0 = *(const float4*)(dx);
            float4 d1 = *(const float4*)(dx + 8);
            float4 d2 = *(const float4*)(dx + 16);
            float4 d3 = *(const float4*)(dx + 24);
            float dxr[16] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w,
                             d2.x, d2.y, d2.z, d2.w, d3.x, d3.y, d3.z, d3.w};
#pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = fmaf((float)isum[r], dw * dxr[r], acc[r]);
        }
#pragma unroll
        for (int r = 0; r < 16; r++) yacc[r] = yacc[r] + acc[r];
    }
    const int col = nt * 64 + wn * 32 + r32;
    if (col >= n) return;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        int row = mt * 64 + wm * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (row < m) {
            size_t o = (size_t)row * ldy + col0 + col;
            float v = yacc[r];
            if (resid) v = resid[o] + v;
            y[o] = v;
        }
    }
}

inline unsigned grid1(size_t n, unsigned block) { return (unsigned)((n + block - 1) / block); }

}  // namespace

// ---- launchers ---------------------------------------------------------------

lq8_status launch_gemv_tile_wg(hipStream_t s, XSource xs, const GemvLaunch& a) {
    if (a.k <= 0 || a.k % 32 || a.n <= 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k must be a positive multiple of 32");
    if (a.k > 16384) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k > 16384 not supported");
    const int nb = a.k / 32, ngroups = (nb + GROUP_BLOCKS - 1) / GROUP_BLOCKS;
    size_t smem = ((size_t)a.k + 4 + (size_t)ngroups * 64) * sizeof(float);
    dim3 grid((unsigned)((a.n + TILE_ROWS - 1) / TILE_ROWS));
    switch (xs) {
        case XS_PLAIN: hipLaunchKernelGGL(k_gemv<XS_PLAIN>, grid, dim3(WG), smem, s, a); break;
        case XS_RMSNORM: hipLaunchKernelGGL(k_gemv<XS_RMSNORM>, grid, dim3(WG), smem, s, a); break;
        case XS_SILU: hipLaunchKernelGGL(k_gemv<XS_SILU>, grid, dim3(WG), smem, s, a); break;
    }
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_gemv_grouped(hipStream_t s, const GemvProblemDev* d_probs, int count, int total_tiles,
                               int max_k) {
    if (count <= 0 || total_tiles <= 0) return LQ8_OK;
    const int ngroups = (max_k / 32 + GROUP_BLOCKS - 1) / GROUP_BLOCKS;
    size_t smem = ((size_t)max_k + 4 + (size_t)ngroups * 64) * sizeof(float);
    hipLaunchKernelGGL(k_gemv_grouped, dim3((unsigned)total_tiles), dim3(WG), smem, s, d_probs, count);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_quantize_act(hipStream_t s, const float* x, int m, int k, int8_t* codes, float* scales32) {
    size_t n = (size_t)m * (k / 32);
    hipLaunchKernelGGL(k_quantize_act, dim3(grid1(n, WG)), dim3(WG), 0, s, x, m, k, codes, scales32);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_quantize_aos(hipStream_t s, const float* x, size_t nblocks, uint8_t* blocks) {
    if (!nblocks) return LQ8_OK;
    hipLaunchKernelGGL(k_quantize_aos, dim3(grid1(nblocks, WG)), dim3(WG), 0, s, x, nblocks, blocks);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_gemm(hipStream_t s, const int8_t* xq, const float* xs, int m, const lq8_weight* w, float* y,
                       const float* resid, int ldy, int col0) {
    dim3 grid((unsigned)w->tiles, (unsigned)((m + 63) / 64));
    hipLaunchKernelGGL(k_gemm, grid, dim3(WG), 0, s, xq, xs, m, w->codes, w->scales, (int)w->n_out, (int)w->nb, y,
                       resid, ldy, col0);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_repack_aos(hipStream_t s, const uint8_t* aos, size_t n_rows, size_t nb, size_t row0,
                             const lq8_weight* w) {
    size_t n = n_rows * nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_repack_aos, dim3(grid1(n, WG)), dim3(WG), 0, s, aos, n_rows, nb, row0, w->codes, w->scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_unpack_aos(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint8_t* aos) {
    size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_unpack_aos, dim3(grid1(n, WG)), dim3(WG), 0, s, w->codes, w->scales, row0, n_rows, w->nb, aos);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_quantize_weight_f32(hipStream_t s, const float* src, size_t n_rows, size_t row0,
                                      const lq8_weight* w) {
    size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_quantize_weight_f32, dim3(grid1(n, WG)), dim3(WG), 0, s, src, n_rows, row0, w->nb, w->codes,
                       w->scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_random_weight(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint64_t seed,
                                uint64_t stream, float stddev) {
    size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    uint64_t key = seed * 0x9E3779B97F4A7C15ull ^ (stream + 1) * 0xC2B2AE3D27D4EB4Full;
    hipLaunchKernelGGL(k_random_weight, dim3(grid1(n, WG)), dim3(WG), 0, s, n_rows, row0, w->nb, key, stddev,
                       w->codes, w->scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_dequant_rows(hipStream_t s, const lq8_weight* w, const uint32_t* d_ids, size_t row0, size_t nrows,
                               float* y) {
    size_t n = nrows * w->k_in;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_dequant_rows, dim3(grid1(n, WG)), dim3(WG), 0, s, w->codes, w->scales, w->nb, d_ids, row0,
                       nrows, y);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

}  // namespace lq8
