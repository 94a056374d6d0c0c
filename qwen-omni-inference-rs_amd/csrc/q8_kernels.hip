// q8_kernels.hip -- Q8_0 format kernels, activation quantization and the
// W8A8 int8-MFMA GEMM for gfx950.
//
// GEMM accumulation order (identical to the CPU oracle, so results are
// bitwise equal): per (m, n), I_b = exact int32 dot of block b from one
// v_mfma_i32_32x32x32_i8; s_b = dw_b * dx_b (exact: two f16 values);
// a_g = fmaf((float)I_b, s_b, a_g) over the blocks of a group of 8, from 0;
// y = y + a_g over the groups, from 0.
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

constexpr int WG = 256;

// Store one quantized block (row, b) into the tiled layout.
__device__ __forceinline__ void store_tiled(int8_t* codes, size_t np, size_t row, size_t b, const int* q) {
    const size_t tile = row / TILE_ROWS;
    const int r = (int)(row % TILE_ROWS);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        w[i] = (uint32_t)(q[4 * i] & 0xFF) | ((uint32_t)(q[4 * i + 1] & 0xFF) << 8) |
               ((uint32_t)(q[4 * i + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * i + 3] & 0xFF) << 24);
    *(uint4*)(codes + code_off(tile, np, b, 0, r)) = make_uint4(w[0], w[1], w[2], w[3]);
    *(uint4*)(codes + code_off(tile, np, b, 1, r)) = make_uint4(w[4], w[5], w[6], w[7]);
}

__device__ __forceinline__ void quantize32(const float* x, int* q, QBlock* qb) {
    const float amax = block_amax(x);
    *qb = block_scale(amax);
    const float id = block_inv(qb->d);
#pragma unroll
    for (int j = 0; j < 32; j++) q[j] = quant_code(x[j], id);
}

// ---- format kernels --------------------------------------------------------

__global__ void k_quantize_weight_f32(const float* __restrict__ src, size_t n_rows, size_t row0, size_t nb, size_t np,
                                      int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const size_t r = idx / nb, b = idx % nb;
    float x[32];
    const float4* s4 = (const float4*)(src + r * nb * 32 + b * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 v = s4[i];
        x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
    }
    int q[32];
    QBlock qb;
    quantize32(x, q, &qb);
    const size_t row = row0 + r;
    store_tiled(codes, np, row, b, q);
    scales[scale_off(row / TILE_ROWS, np, b, (int)(row % TILE_ROWS))] = qb.d16;
}

__global__ void k_quantize_aos(const float* __restrict__ src, size_t nblocks, uint8_t* __restrict__ dst) {
    const size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
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

__global__ void k_repack_aos(const uint8_t* __restrict__ aos, size_t n_rows, size_t nb, size_t np, size_t row0,
                             int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const size_t r = idx / nb, b = idx % nb;
    const uint8_t* blk = aos + idx * BLOCK_BYTES;
    int q[32];
#pragma unroll
    for (int j = 0; j < 32; j++) q[j] = (int)(int8_t)blk[2 + j];
    const size_t row = row0 + r;
    store_tiled(codes, np, row, b, q);
    scales[scale_off(row / TILE_ROWS, np, b, (int)(row % TILE_ROWS))] = (uint16_t)(blk[0] | (blk[1] << 8));
}

__global__ void k_unpack_aos(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales, size_t row0,
                             size_t n_rows, size_t nb, size_t np, uint8_t* __restrict__ aos) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const size_t row = row0 + idx / nb, b = idx % nb;
    const size_t tile = row / TILE_ROWS;
    const int r = (int)(row % TILE_ROWS);
    uint8_t* o = aos + idx * BLOCK_BYTES;
    const uint16_t d = scales[scale_off(tile, np, b, r)];
    o[0] = (uint8_t)(d & 0xFF);
    o[1] = (uint8_t)(d >> 8);
    const int8_t* lo = codes + code_off(tile, np, b, 0, r);
    const int8_t* hi = codes + code_off(tile, np, b, 1, r);
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
__global__ void k_random_weight(size_t n_rows, size_t row0, size_t nb, size_t np, uint64_t key, float stddev,
                                int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const size_t r = idx / nb, b = idx % nb;
    const size_t row = row0 + r;
    float x[32];
    const size_t pair0 = (r * nb * 32 + b * 32) / 2;
#pragma unroll 4
    for (int i = 0; i < 16; i++) {
        const uint64_t h = splitmix64(key + (pair0 + i) * 0xD1B54A32D192ED03ull);
        const float u1 = ((float)(uint32_t)(h >> 40) + 1.0f) * 5.9604644775390625e-8f;
        const float u2 = (float)(uint32_t)((h >> 16) & 0xFFFFFFu) * 5.9604644775390625e-8f;
        const float rad = sqrtf(-2.0f * logf(u1));
        const float th = 6.283185307179586f * u2;
        x[2 * i] = stddev * rad * cosf(th);
        x[2 * i + 1] = stddev * rad * sinf(th);
    }
    int q[32];
    QBlock qb;
    quantize32(x, q, &qb);
    store_tiled(codes, np, row, b, q);
    scales[scale_off(row / TILE_ROWS, np, b, (int)(row % TILE_ROWS))] = qb.d16;
}

// y[i, c] = d * q for rows ids[i] (or row0 + i when ids is null): exact.
__global__ void k_dequant_rows(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales, size_t nb,
                               size_t np, const uint32_t* __restrict__ ids, size_t row0, size_t nrows,
                               float* __restrict__ y) {
    const size_t k = nb * 32;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= nrows * k) return;
    const size_t i = idx / k, c = idx % k;
    const size_t row = ids ? (size_t)ids[i] : row0 + i;
    const size_t tile = row / TILE_ROWS, b = c / 32;
    const int r = (int)(row % TILE_ROWS), j = (int)(c % 32);
    const float d = f16_bits_to_f32(scales[scale_off(tile, np, b, r)]);
    const int8_t q = codes[code_off(tile, np, b, j >> 4, r) + (j & 15)];
    y[idx] = d * (float)q;
}

// ---- activation quantization (tiled A operand of the GEMM) ----------------

__global__ void k_quantize_act(const float* __restrict__ x, int m, int k, int8_t* __restrict__ codes,
                               float* __restrict__ scales32) {
    const size_t nb = (size_t)k / 32, np = (nb + 1) / 2;
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)m * nb) return;
    const size_t r = idx / nb, b = idx % nb;
    float v[32];
    const float4* s4 = (const float4*)(x + r * (size_t)k + b * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 t = s4[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    int q[32];
    QBlock qb;
    quantize32(v, q, &qb);
    store_tiled(codes, np, r, b, q);
    scales32[scale_off(r / TILE_ROWS, np, b, (int)(r % TILE_ROWS))] = f16_bits_to_f32(qb.d16);
}

// ---- GEMM (W8A8, v_mfma_i32_32x32x32_i8) -------------------------------------

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// Workgroup tile 64 (m) x 64 (n); wave w owns the 32 x 32 sub-tile (w >> 1, w & 1).
// Operand lane l of a 32-row MFMA tile at row R0: row R0 + l % 32 (16-row tile
// R0 / 16 + (l % 32) / 16), codes of half l / 32 of the block; the two operands
// use the same split of the 32 k-values, so the int32 block dot is exact.
// Accumulator layout: lane l holds column l % 32, register i holds row
// 8 * (i / 4) + 4 * (l / 32) + i % 4.
__global__ __launch_bounds__(WG) void k_gemm(const int8_t* __restrict__ xq, const float* __restrict__ xs32, int m,
                                             const int8_t* __restrict__ wc, const uint16_t* __restrict__ ws, int n,
                                             int nb, float* __restrict__ y, const float* __restrict__ resid) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int mt32 = blockIdx.y * 2 + (wave >> 1), nt32 = blockIdx.x * 2 + (wave & 1);
    if (mt32 * 32 >= m || nt32 * 32 >= n) return;  // no barriers below
    const int np = (nb + 1) >> 1;
    const int half = lane >> 5, r32 = lane & 31;
    const int atile = mt32 * 2 + (r32 >> 4), btile = nt32 * 2 + (r32 >> 4);
    const int8_t* ab = xq + ((size_t)atile * np * 64 + half * 16 + (r32 & 15)) * 16;
    const int8_t* bb = wc + ((size_t)btile * np * 64 + half * 16 + (r32 & 15)) * 16;
    // scale pointers: dw for column r32 (tile btile, row r32 % 16); dx rows 4*half + 0..3 (+8) in tiles 2*mt32, 2*mt32+1
    const uint16_t* dwp = ws + (size_t)btile * 2 * np * 16 + (r32 & 15);
    const float* dxp0 = xs32 + (size_t)(mt32 * 2) * 2 * np * 16 + 4 * half;
    const float* dxp1 = xs32 + (size_t)(mt32 * 2 + 1) * 2 * np * 16 + 4 * half;
    auto boff = [&](int b) { return (size_t)((b >> 1) * 64 + (b & 1) * 32) * 16; };
    float yacc[16], acc[16];
#pragma unroll
    for (int i = 0; i < 16; i++) { yacc[i] = 0.0f; acc[i] = 0.0f; }
    const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    v4i av = *(const v4i*)(ab + boff(0));
    v4i bv = *(const v4i*)(bb + boff(0));
    for (int b = 0; b < nb; b++) {
        const v4i a_cur = av, b_cur = bv;
        if (b + 1 < nb) {
            av = *(const v4i*)(ab + boff(b + 1));
            bv = *(const v4i*)(bb + boff(b + 1));
        }
        const float dw = f16_bits_to_f32(dwp[b * 16]);
        const float4 d0 = *(const float4*)(dxp0 + b * 16);
        const float4 d1 = *(const float4*)(dxp0 + b * 16 + 8);
        const float4 d2 = *(const float4*)(dxp1 + b * 16);
        const float4 d3 = *(const float4*)(dxp1 + b * 16 + 8);
        const float dx[16] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w,
                              d2.x, d2.y, d2.z, d2.w, d3.x, d3.y, d3.z, d3.w};
        const v16i isum = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur, b_cur, zero, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = fmaf((float)isum[i], dw * dx[i], acc[i]);
        if ((b % GEMM_GROUP) == GEMM_GROUP - 1 || b == nb - 1) {
#pragma unroll
            for (int i = 0; i < 16; i++) { yacc[i] = yacc[i] + acc[i]; acc[i] = 0.0f; }
        }
    }
    const int col = nt32 * 32 + r32;
    if (col >= n) return;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int row = mt32 * 32 + 8 * (i >> 2) + 4 * half + (i & 3);
        if (row < m) {
            const size_t o = (size_t)row * n + col;
            float v = yacc[i];
            if (resid) v = resid[o] + v;
            y[o] = v;
        }
    }
}

inline unsigned grid1(size_t n, unsigned block) { return (unsigned)((n + block - 1) / block); }

}  // namespace

// ---- launchers ---------------------------------------------------------------

size_t act_code_bytes(int m, int k) {
    const size_t np = ((size_t)k / 32 + 1) / 2;
    return (size_t)((m + 31) / 32) * 2 * np * CHUNK_BYTES;
}
size_t act_scale_bytes(int m, int k) {
    const size_t np = ((size_t)k / 32 + 1) / 2;
    return (size_t)((m + 31) / 32) * 2 * 2 * np * 16 * sizeof(float);
}

lq8_status launch_quantize_act(hipStream_t s, const float* x, int m, int k, int8_t* codes, float* scales32) {
    const size_t n = (size_t)m * (k / 32);
    if (!n) return LQ8_OK;
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
                       const float* resid) {
    const dim3 grid((unsigned)((w->n_out + 63) / 64), (unsigned)((m + 63) / 64));
    hipLaunchKernelGGL(k_gemm, grid, dim3(WG), 0, s, xq, xs, m, w->codes, w->scales, (int)w->n_out, (int)w->nb, y,
                       resid);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_repack_aos(hipStream_t s, const uint8_t* aos, size_t n_rows, size_t row0, const lq8_weight* w) {
    const size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_repack_aos, dim3(grid1(n, WG)), dim3(WG), 0, s, aos, n_rows, w->nb, w->np, row0, w->codes,
                       w->scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_unpack_aos(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint8_t* aos) {
    const size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_unpack_aos, dim3(grid1(n, WG)), dim3(WG), 0, s, w->codes, w->scales, row0, n_rows, w->nb,
                       w->np, aos);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_quantize_weight_f32(hipStream_t s, const float* src, size_t n_rows, size_t row0,
                                      const lq8_weight* w) {
    const size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_quantize_weight_f32, dim3(grid1(n, WG)), dim3(WG), 0, s, src, n_rows, row0, w->nb, w->np,
                       w->codes, w->scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_random_weight(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint64_t seed,
                                uint64_t stream, float stddev) {
    const size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    const uint64_t key = seed * 0x9E3779B97F4A7C15ull ^ (stream + 1) * 0xC2B2AE3D27D4EB4Full;
    hipLaunchKernelGGL(k_random_weight, dim3(grid1(n, WG)), dim3(WG), 0, s, n_rows, row0, w->nb, w->np, key, stddev,
                       w->codes, w->scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_dequant_rows(hipStream_t s, const lq8_weight* w, const uint32_t* d_ids, size_t row0, size_t nrows,
                               float* y) {
    const size_t n = nrows * w->k_in;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_dequant_rows, dim3(grid1(n, WG)), dim3(WG), 0, s, w->codes, w->scales, w->nb, w->np, d_ids,
                       row0, nrows, y);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

}  // namespace lq8
