// q8_kernels.hip -- Q8_0 format kernels, activation quantization and the
// W8A8 int8-MFMA GEMM for gfx950.
//
// GEMM accumulation order (identical to the CPU oracle, so results are
// bitwise equal): per (m, n), I_b = exact int32 dot of block b from one
// v_mfma_i32_32x32x32_i8; s_b = dw_b * dx_b (exact: two f16 values);
// a_g = fmaf((float)I_b, s_b, a_g) over the blocks of a group of 8, from 0;
// y = y + a_g over the groups, from 0.
#include <algorithm>

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
                             RowRun rr, int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const size_t r = idx / nb, b = idx % nb;
    const uint8_t* blk = aos + idx * BLOCK_BYTES;
    int q[32];
#pragma unroll
    for (int j = 0; j < 32; j++) q[j] = (int)(int8_t)blk[2 + j];
    const size_t row = map_row(row0, r, rr);
    store_tiled(codes, np, row, b, q);
    scales[scale_off(row / TILE_ROWS, np, b, (int)(row % TILE_ROWS))] = (uint16_t)(blk[0] | (blk[1] << 8));
}

__global__ void k_unpack_aos(const int8_t* __restrict__ codes, const uint16_t* __restrict__ scales, size_t row0,
                             RowRun rr, size_t n_rows, size_t nb, size_t np, uint8_t* __restrict__ aos) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const size_t row = map_row(row0, idx / nb, rr), b = idx % nb;
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

// The GEMM's activation operand (tiled codes, f16 scales in the operand
// layout [m/32][2 groups][64 lanes][4 blocks]) back to GGUF blocks, one
// thread per (row, block).
__global__ void k_unpack_act(const int8_t* __restrict__ codes, const uint32_t* __restrict__ xs, int m, int nb, int np,
                             int nbp4, uint8_t* __restrict__ aos) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)m * nb) return;
    const int row = (int)(idx / nb), b = (int)(idx % nb);
    const uint32_t d = xs[((size_t)((row >> 5) * nbp4 + (b >> 2)) * 64 + (row & 31)) * 4 + (b & 3)];
    uint8_t* o = aos + idx * BLOCK_BYTES;
    o[0] = (uint8_t)(d & 0xFF);
    o[1] = (uint8_t)((d >> 8) & 0xFF);
    const int8_t* lo = codes + code_off(row / TILE_ROWS, np, b, 0, row % TILE_ROWS);
    const int8_t* hi = codes + code_off(row / TILE_ROWS, np, b, 1, row % TILE_ROWS);
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
__global__ void k_random_weight(size_t n_rows, size_t row0, RowRun rr, size_t nb, size_t np, uint64_t key,
                                float stddev, int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const size_t r = idx / nb, b = idx % nb;  // the values depend on (r, b), not on where row r is stored
    const size_t row = map_row(row0, r, rr);
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

// bf16 rows (checkpoint weights) -> the tiled Q8_0 layout; a bf16 value is
// exactly the f32 with those 16 high bits, so this is the f32 quantizer on
// the widened values.
__global__ void k_quantize_weight_bf16(const uint16_t* __restrict__ src, size_t n_rows, size_t row0, size_t nb,
                                       size_t np, int8_t* __restrict__ codes, uint16_t* __restrict__ scales) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n_rows * nb) return;
    const size_t r = idx / nb, b = idx % nb;
    float x[32];
    const uint4* s4 = (const uint4*)(src + r * nb * 32 + b * 32);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 v = s4[i];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            x[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
            x[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
        }
    }
    int q[32];
    QBlock qb;
    quantize32(x, q, &qb);
    const size_t row = row0 + r;
    store_tiled(codes, np, row, b, q);
    scales[scale_off(row / TILE_ROWS, np, b, (int)(row % TILE_ROWS))] = qb.d16;
}

// ---- activation quantization (tiled A operand of the GEMM) ----------------

// One wave per (16-row tile, block pair): its 64 lanes write the pair's 1 KiB
// code chunk with one 16-byte store each.  Lane l covers row l % 16 of the
// tile and part l / 16 of the chunk, i.e. half (l / 16) % 2 of block
// 2p + l / 32; the two halves of a block (lanes l and l ^ 16) share amax
// through one shuffle (max is exact in any order).  Rows past m repeat row
// m - 1 (finite data for the padding rows of the last 32-row tile); blocks
// past nb get zero codes and a zero scale.  Scales go to the GEMM's f16
// operand layout: u32 words (f16 bits, high half zero) in
// [m/32][nbp/4][64 lanes][4 blocks], lanes 0..31 = rows, lanes 32..63 = 0.
// amax of 16 values from 0, NaN ignored (as `if (v > amax) amax = v`):
// fmaxf returns the non-NaN operand.
__device__ __forceinline__ float half_amax(const float* v) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[i]));
    return amax;
}

// Store half hf of block b of activation row `row`: the 16 codes of v under the
// block's amax (both halves combined) into the tiled code layout (only where a
// code slot exists, b < 2 np; zero codes past nb), and into the scale layout
// [m/32][nbp/4][64 lanes][4 blocks] the f16 scale (half 0; 0 past nb) or the
// zero of the upper 32 lanes (half 1).
__device__ __forceinline__ void put_act_half(int8_t* __restrict__ codes, uint32_t* __restrict__ xs, int np, int nbp4,
                                             int nb, int row, int b, int hf, const float* v, float amax) {
    uint32_t d16 = 0;
    if (b < 2 * np) {
        uint4 c = make_uint4(0, 0, 0, 0);
        if (b < nb) {
            const QBlock qb = block_scale(amax);
            const float id = block_inv(qb.d);
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                w[i] = (uint32_t)(quant_code(v[4 * i], id) & 0xFF) |
                       ((uint32_t)(quant_code(v[4 * i + 1], id) & 0xFF) << 8) |
                       ((uint32_t)(quant_code(v[4 * i + 2], id) & 0xFF) << 16) |
                       ((uint32_t)(quant_code(v[4 * i + 3], id) & 0xFF) << 24);
            c = make_uint4(w[0], w[1], w[2], w[3]);
            d16 = qb.d16;
        }
        *(uint4*)(codes + code_off(row / TILE_ROWS, np, b, hf, row % TILE_ROWS)) = c;
    }
    xs[((size_t)((row >> 5) * nbp4 + (b >> 2)) * 64 + hf * 32 + (row & 31)) * 4 + (b & 3)] = hf ? 0u : d16;
}

__global__ __launch_bounds__(256) void k_quantize_act(const float* __restrict__ x, int m, int k, int waves, int np8,
                                                      int8_t* __restrict__ codes, uint32_t* __restrict__ xs) {
    const int gw = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (gw >= waves) return;
    const int lane = threadIdx.x & 63;
    const int tile = gw / np8, p = gw - tile * np8;
    const int nb = k >> 5, np = (nb + 1) >> 1;
    const int r = lane & 15, part = lane >> 4, b = 2 * p + (part >> 1), hf = part & 1;
    float v[16] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    float amax = 0.0f;
    if (p < np) {
        const int row = min(tile * TILE_ROWS + r, m - 1);
        const float4* src = (const float4*)(x + (size_t)row * k + min(b, nb - 1) * 32 + hf * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = src[i];
            v[4 * i] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
        amax = half_amax(v);
        amax = fmaxf(amax, lane_xor<16>(amax));
    }
    put_act_half(codes, xs, np, np8 >> 1, nb, tile * TILE_ROWS + r, b, hf, v, amax);
}

// RMSNorm of rows x[m, dim] quantized straight into the GEMM operand layout:
// the same values as k_quantize_act applied to the output of
// k_rms_norm_rows (SUM64 of bf16(x)^2, mean = sum / dim,
// inv = 1 / sqrt(mean + eps), out = bf16((bf16(x) * inv) * bf16(w)),
// src/rms_norm.rs:143-176).  One wave per padded row (rows past m repeat row
// m - 1); lane l holds elements l, l + 64, ... in registers for the sum,
// the normed row is staged in LDS, then lane l quantizes half-blocks l,
// l + 64, ... (16 consecutive values each; the two halves of a block are
// neighbouring lanes).  dim <= 64 U.
template <int U>
__global__ __launch_bounds__(256) void k_rms_quantize_act(const float* __restrict__ x, const float* __restrict__ w, int m,
                                                          int dim, float eps, int np, int nbp,
                                                          int8_t* __restrict__ codes, uint32_t* __restrict__ xs) {
    __shared__ __attribute__((aligned(16))) float rowbuf[4][64 * U];
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wv;  // the grid covers the padded rows exactly
    const float* xr = x + (size_t)min(row, m - 1) * dim;
    float v[U], wn[U];  // the norm weights are loaded with the row, off the sum's critical path
#pragma unroll
    for (int u = 0; u < U; u++) {
        v[u] = xr[min(lane + 64 * u, dim - 1)];
        wn[u] = w[min(lane + 64 * u, dim - 1)];
    }
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < U; u++)
        if (lane + 64 * u < dim) {
            const float b = bf16_round(v[u]);
            acc = acc + b * b;
        }
    acc = wave_sum64(acc);
    const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)dim) + eps));
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int i = lane + 64 * u;
        if (i < dim) rowbuf[wv][i] = bf16_round((bf16_round(v[u]) * inv) * bf16_round(wn[u]));
    }
    __syncthreads();
    const int nb = dim >> 5, nhb = 2 * nbp;
    for (int hb0 = 0; hb0 < nhb; hb0 += 64) {
        const int hb = hb0 + lane, b = hb >> 1, hf = hb & 1;
        float q[16] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        if (b < nb) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 t = *(const float4*)&rowbuf[wv][b * 32 + hf * 16 + 4 * i];
                q[4 * i] = t.x;
                q[4 * i + 1] = t.y;
                q[4 * i + 2] = t.z;
                q[4 * i + 3] = t.w;
            }
        }
        float amax = half_amax(q);
        amax = fmaxf(amax, lane_xor<1>(amax));
        if (hb < nhb) put_act_half(codes, xs, np, nbp >> 2, nb, row, b, hf, q, amax);
    }
}

// Routed expert outputs combined into the hidden state, then RMSNorm'd and
// quantized for the next layer's q|k|v GEMM: one workgroup of 1024 threads
// per padded row (rows past m repeat row m - 1 and write only the operand);
// a thread loads its elements of every routed expert up front.  The combine is
// k_moe_combine's arithmetic (acc = acc + w * y over the token's experts in
// ascending index, from 0; h = h2 + acc), written to out for rows < m; the
// rest is k_rms_quantize_act's on h (bf16(h)^2 summed in the SUM64 order by
// wave 0, normed row staged in LDS, half-blocks quantized by neighbouring
// lanes).  dim <= CRQ_MAX_DIM.
constexpr int CRQ_MAX_DIM = 2048, CRQ_MAX_K = 16, CRQ_THREADS = 1024, CRQ_PER = CRQ_MAX_DIM / CRQ_THREADS;

__global__ __launch_bounds__(CRQ_THREADS) void k_combine_rms_quant(
    const float* __restrict__ h2, const float* __restrict__ eo, const uint32_t* __restrict__ rids,
    const float* __restrict__ rw, int K, int m, int dim, const float* __restrict__ w, float eps, int np, int nbp,
    float* __restrict__ out, int8_t* __restrict__ codes, uint32_t* __restrict__ xs) {
    __shared__ __attribute__((aligned(16))) float hrow[CRQ_MAX_DIM];
    __shared__ int order[CRQ_MAX_K];
    __shared__ float inv_s;
    const int row = blockIdx.x, t = min(row, m - 1), tid = threadIdx.x;
    float hv[CRQ_PER], wn[CRQ_PER];  // the norm weights load with the row, off the critical path
#pragma unroll
    for (int e = 0; e < CRQ_PER; e++) {
        const int ic = min(tid + e * CRQ_THREADS, dim - 1);
        hv[e] = h2[(size_t)t * dim + ic];
        wn[e] = w[ic];
    }
    if (tid < K) {
        const uint32_t me = rids[t * K + tid];
        int below = 0;
        for (int r = 0; r < K; r++) below += rids[t * K + r] < me;
        order[below] = tid;  // expert ids of a token are distinct
    }
    __syncthreads();
    // every load of the row's experts in flight before the sums
    float wv[CRQ_MAX_K], ev[CRQ_PER][CRQ_MAX_K];
#pragma unroll
    for (int q = 0; q < CRQ_MAX_K; q++) {
        if (q < K) {
            const int slot = t * K + order[q];
            wv[q] = rw[slot];
#pragma unroll
            for (int e = 0; e < CRQ_PER; e++) ev[e][q] = eo[(size_t)slot * dim + min(tid + e * CRQ_THREADS, dim - 1)];
        }
    }
#pragma unroll
    for (int e = 0; e < CRQ_PER; e++) {
        const int i = tid + e * CRQ_THREADS;
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < CRQ_MAX_K; q++)
            if (q < K) acc = acc + wv[q] * ev[e][q];
        const float h = hv[e] + acc;
        if (i < dim) {
            if (row < m) out[(size_t)t * dim + i] = h;
            hrow[i] = h;
        }
    }
    __syncthreads();
    if (tid < 64) {
        float v[CRQ_MAX_DIM / 64];  // every LDS read in flight, then the adds in order
#pragma unroll
        for (int u = 0; u < CRQ_MAX_DIM / 64; u++) v[u] = hrow[min(tid + 64 * u, dim - 1)];
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < CRQ_MAX_DIM / 64; u++)
            if (tid + 64 * u < dim) {
                const float b = bf16_round(v[u]);
                acc = acc + b * b;
            }
        acc = wave_sum64(acc);
        if (tid == 0) inv_s = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)dim) + eps));
    }
    __syncthreads();
    const float inv = inv_s;
#pragma unroll
    for (int e = 0; e < CRQ_PER; e++) {
        const int i = tid + e * CRQ_THREADS;
        if (i < dim) hrow[i] = bf16_round((bf16_round(hrow[i]) * inv) * bf16_round(wn[e]));
    }
    __syncthreads();
    const int nb = dim >> 5, nhb = 2 * nbp;
    for (int hb0 = 0; hb0 < nhb; hb0 += CRQ_THREADS) {
        const int hb = hb0 + tid, b = hb >> 1, hf = hb & 1;
        float q[16] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        if (b < nb) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v4 = *(const float4*)&hrow[b * 32 + hf * 16 + 4 * i];
                q[4 * i] = v4.x;
                q[4 * i + 1] = v4.y;
                q[4 * i + 2] = v4.z;
                q[4 * i + 3] = v4.w;
            }
        }
        float amax = half_amax(q);
        amax = fmaxf(amax, lane_xor<1>(amax));
        if (hb < nhb) put_act_half(codes, xs, np, nbp >> 2, nb, row, b, hf, q, amax);
    }
}

// act = silu(gate) * up of rows gu[m, 2 inter] (as k_silu_mul: silu(g) =
// g / (1 + exp(-g)), src/tensor.rs:1978, mlp.rs:151-164) quantized straight
// into the GEMM operand layout.  One wave per (padded row, group of 8
// blocks): lanes 8j .. 8j + 7 hold block j of the group, 4 consecutive values
// each (lanes 8j .. 8j + 3 half 0, 8j + 4 .. 8j + 7 half 1); the block amax
// folds over those 8 lanes (max is exact in any order).  Rows past m repeat
// row m - 1.
__global__ __launch_bounds__(256) void k_silu_quantize_act(const float* __restrict__ gu, int m, int inter, int waves,
                                                           int groups, int np, int8_t* __restrict__ codes,
                                                           uint32_t* __restrict__ xs) {
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (gw >= waves) return;
    const int lane = threadIdx.x & 63;
    const int row = gw / groups, g = gw - row * groups;
    const int b = g * GEMM_GROUP + (lane >> 3), hf = (lane >> 2) & 1, sub = lane & 3, nb = inter >> 5;
    float q[4] = {0, 0, 0, 0};
    if (b < nb) {
        const float* gp = gu + (size_t)min(row, m - 1) * 2 * inter + b * 32 + hf * 16 + sub * 4;
        const float4 gv = *(const float4*)gp, uv = *(const float4*)(gp + inter);
        q[0] = __fdiv_rn(gv.x, 1.0f + expf_cr(-gv.x)) * uv.x;
        q[1] = __fdiv_rn(gv.y, 1.0f + expf_cr(-gv.y)) * uv.y;
        q[2] = __fdiv_rn(gv.z, 1.0f + expf_cr(-gv.z)) * uv.z;
        q[3] = __fdiv_rn(gv.w, 1.0f + expf_cr(-gv.w)) * uv.w;
    }
    float amax = fmaxf(fmaxf(fmaxf(0.0f, fabsf(q[0])), fabsf(q[1])), fmaxf(fabsf(q[2]), fabsf(q[3])));
    amax = fmaxf(amax, lane_xor<1>(amax));
    amax = fmaxf(amax, lane_xor<2>(amax));
    amax = fmaxf(amax, lane_xor<4>(amax));
    uint32_t d16 = 0;
    if (b < 2 * np) {
        uint32_t c = 0;
        if (b < nb) {
            const QBlock qb = block_scale(amax);
            const float id = block_inv(qb.d);
            c = (uint32_t)(quant_code(q[0], id) & 0xFF) | ((uint32_t)(quant_code(q[1], id) & 0xFF) << 8) |
                ((uint32_t)(quant_code(q[2], id) & 0xFF) << 16) | ((uint32_t)(quant_code(q[3], id) & 0xFF) << 24);
            d16 = qb.d16;
        }
        *(uint32_t*)(codes + code_off(row / TILE_ROWS, np, b, hf, row % TILE_ROWS) + 4 * sub) = c;
    }
    if (sub == 0)
        xs[((size_t)((row >> 5) * 2 * groups + (b >> 2)) * 64 + hf * 32 + (row & 31)) * 4 + (b & 3)] = hf ? 0u : d16;
}

// Attention outputs of one (head, sequence) combined from the segment
// partials (the arithmetic of k_attn_combine, thread by thread) and quantized
// straight into the GEMM operand layout (the values k_quantize_act gives for
// those outputs): 128 threads, thread d element d of the head; the head's 4
// blocks are 8 half-blocks, which threads 0..7 quantize from LDS (the two
// halves of a block are neighbouring threads).  The workgroup of the last
// head also writes the zero scales of the padding blocks past nb (the GEMM
// reads them with the block's quad).
__global__ __launch_bounds__(128) void k_attn_combine_quant(const float* __restrict__ part, size_t part_stride,
                                                            const int* __restrict__ d_pos, int H, int cmax, int np,
                                                            int nbp4, int8_t* __restrict__ codes,
                                                            uint32_t* __restrict__ xs) {
    __shared__ __attribute__((aligned(16))) float o[128];
    const int h = blockIdx.x, row = blockIdx.y, d = threadIdx.x;
    const float* pb = part + row * part_stride;
    // the first CQ segments' partials load with the position (indices
    // clamped to the capacity: in bounds, entries past the position unused)
    constexpr int CQ = 4;
    float mq[CQ], lq[CQ], oq[CQ];
#pragma unroll
    for (int c = 0; c < CQ; c++) {
        const float* p = pb + ((size_t)min(c, cmax - 1) * H + h) * ATT_PART_STRIDE;
        mq[c] = p[128];
        lq[c] = p[129];
        oq[c] = p[d];
    }
    const int C = min(max(d_pos[row], 0) / ATT_SEG + 1, cmax);
    float m = -__builtin_huge_valf(), den = 0.0f, num = 0.0f;
    for (int c = 0; c < C; c++) {
        float mc, lc, oc;
        if (c < CQ) {
            mc = mq[c];
            lc = lq[c];
            oc = oq[c];
        } else {
            const float* p = pb + ((size_t)c * H + h) * ATT_PART_STRIDE;
            mc = p[128];
            lc = p[129];
            oc = p[d];
        }
        const float mn = m > mc ? m : mc;
        const float ea = expf_cr(m - mn), eb = expf_cr(mc - mn);
        den = den * ea + eb * lc;
        num = num * ea + eb * oc;
        m = mn;
    }
    o[d] = __fdiv_rn(num, den);
    __syncthreads();
    const int nb = H * 4;
    if (d < 8) {
        const int hf = d & 1, b = h * 4 + (d >> 1);
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = *(const float4*)&o[(d >> 1) * 32 + hf * 16 + 4 * i];
            v[4 * i] = t.x;
            v[4 * i + 1] = t.y;
            v[4 * i + 2] = t.z;
            v[4 * i + 3] = t.w;
        }
        float amax = half_amax(v);
        amax = fmaxf(amax, lane_xor<1>(amax));
        put_act_half(codes, xs, np, nbp4, nb, row, b, hf, v, amax);
    }
    if (h == H - 1) {
        // padding blocks nb .. 4 nbp4 - 1: zero scale words (both halves)
        for (int i = d; i < 2 * (4 * nbp4 - nb); i += 128) {
            const int b = nb + (i >> 1), hf = i & 1;
            xs[((size_t)((row >> 5) * nbp4 + (b >> 2)) * 64 + hf * 32 + (row & 31)) * 4 + (b & 3)] = 0u;
        }
    }
}

// ---- GEMM (W8A8, v_mfma_i32_32x32x32_i8) -------------------------------------

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

constexpr int RSRC_CFG = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

struct GemmArgs {
    const int8_t* xq;   // activation codes, tiled like a weight (2 * ntm 16-row tiles)
    const uint32_t* xs; // activation scales, f16 operand layout written by k_quantize_act
    const int8_t* wc;   // weight codes
    const uint16_t* ws; // weight scales (f16 bits)
    float* y;
    const float* resid;
    int m, n, nb, np, groups, ntm, ntiles;
    int xq_bytes, xs_bytes, wc_bytes, ws_bytes;
};

// Buffer resources and per-lane byte offsets of one wave's operands: TM
// activation m-tiles and TN weight n-tiles of 32 rows each.
template <int TM, int TN>
struct GemmSrc {
    __amdgpu_buffer_rsrc_t ra, rb, rx, rw;
    int oa[TM], ob[TN], ox[TM], ow[TN];
};

// Operands of 4 consecutive blocks b0 .. b0 + 3 (b0 % 4 == 0) for a TM x TN
// wave tile.  Codes and weight scales of blocks past nb are read from block
// nb - 1 (in bounds); their products are cancelled by zero scales in the
// compute step.
template <int TM, int TN>
struct Quad {
    v4i dx[TM];   // activation scales of the 4 blocks (lanes 32..63: 0)
    v4i a[TM][4], w[TN][4];
    uint32_t dw[TN][4];
};

template <int TM, int TN>
__device__ __forceinline__ void gemm_load(const GemmSrc<TM, TN>& o, int b0, int nb, Quad<TM, TN>& q) {
#pragma unroll
    for (int t = 0; t < TM; t++)
        q.dx[t] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(o.rx, o.ox[t], (b0 >> 2) * 1024, 0));
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int bc = min(b0 + i, nb - 1);
        const int cs = (bc >> 1) * 1024 + (bc & 1) * 512;
#pragma unroll
        for (int t = 0; t < TM; t++)
            q.a[t][i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(o.ra, o.oa[t], cs, 0));
#pragma unroll
        for (int t = 0; t < TN; t++) {
            q.w[t][i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(o.rb, o.ob[t], cs, 0));
            q.dw[t][i] = __builtin_amdgcn_raw_buffer_load_b16(o.rw, o.ow[t], bc * 32, 0);
        }
    }
}

// acc[tile][r] = fmaf((float)I_b[r], dw_b * dx_b[r], acc[tile][r]) for the 4
// blocks in order, for every (m, n) tile of the wave.  The scale products
// come from one v_mfma_f32_32x32x8f16 per block and tile: A = (dx[row], 0, 0,
// 0) in lanes 0..31 and 0 in lanes 32..63, B = (dw[col], 0, 0, 0) in lanes
// 0..31 of a real block and 0 elsewhere, so D[row][col] = dx * dw exactly (a
// product of two f16 values fits f32) -- the same value the VALU product
// gives -- and exactly 0 for a block past nb.
template <int TM, int TN>
__device__ __forceinline__ void gemm_quad(const Quad<TM, TN>& q, int b0, int nb, bool lo, float (*acc)[16]) {
    const v16i zi = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
#pragma unroll
            for (int tn = 0; tn < TN; tn++) {
                const v16i I = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.a[tm][i], q.w[tn][i], zi, 0, 0, 0);
                const uint2 au = {(uint32_t)q.dx[tm][i], 0u};
                const uint2 bu = {(lo && b0 + i < nb) ? q.dw[tn][i] : 0u, 0u};
                const v16f P = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, au),
                                                                    __builtin_bit_cast(v4h, bu), zf, 0, 0, 0);
                float* a = acc[tm * TN + tn];
#pragma unroll
                for (int r = 0; r < 16; r++) a[r] = fmaf((float)I[r], P[r], a[r]);
            }
        }
    }
}

// One round: the wave's group g (8 blocks in two quads q0, q1), with the
// loads of the next round's group gn issued behind each quad's compute.
template <bool NEXT, int TM, int TN>
__device__ __forceinline__ void gemm_group(const GemmSrc<TM, TN>& o, int g, int gn, int nb, bool lo,
                                           Quad<TM, TN>& q0, Quad<TM, TN>& q1, float (*acc)[16]) {
#pragma unroll
    for (int t = 0; t < TM * TN; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    gemm_quad(q0, g * GEMM_GROUP, nb, lo, acc);
    if (NEXT) gemm_load(o, gn * GEMM_GROUP, nb, q0);
    gemm_quad(q1, g * GEMM_GROUP + 4, nb, lo, acc);
    if (NEXT) gemm_load(o, gn * GEMM_GROUP + 4, nb, q1);
}

// Round combine: wave 0 adds its own group, then the other waves' groups
// from LDS, in group order (y = y + a_g).  Two barriers: the partials are
// written, read, and free again before the next round writes them.
template <int S, int T, bool ONE>
__device__ __forceinline__ void gemm_combine(float4* part, int j, int s, int lane, int G, float (*acc)[16],
                                             float (*y)[16]) {
    if (S == 1) {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) y[t][r] = (ONE ? 0.0f : y[t][r]) + acc[t][r];
        return;
    }
    if (s > 0 && j * S + s < G) {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int q = 0; q < 4; q++)
                part[(((s - 1) * T + t) * 4 + q) * 64 + lane] =
                    make_float4(acc[t][4 * q], acc[t][4 * q + 1], acc[t][4 * q + 2], acc[t][4 * q + 3]);
    }
    __syncthreads();
    if (s == 0) {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) y[t][r] = (ONE ? 0.0f : y[t][r]) + acc[t][r];
        for (int u = 1; u < S && j * S + u < G; u++) {
#pragma unroll
            for (int t = 0; t < T; t++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 v = part[(((u - 1) * T + t) * 4 + q) * 64 + lane];
                    y[t][4 * q] = y[t][4 * q] + v.x;
                    y[t][4 * q + 1] = y[t][4 * q + 1] + v.y;
                    y[t][4 * q + 2] = y[t][4 * q + 2] + v.z;
                    y[t][4 * q + 3] = y[t][4 * q + 3] + v.w;
                }
        }
    }
    __syncthreads();
}

// One (32 TM) x (32 TN) output block per workgroup of S waves, as TM x TN
// MFMA tiles of 32 x 32 that share each fetched operand fragment (a weight
// fragment serves TM tiles, an activation fragment TN); wave s takes the
// groups g = s, s + S, s + 2S, ... (one per round).  Blocks are numbered so
// that the workgroups one XCD receives (workgroup ids congruent mod 8) cover
// a contiguous run of n-blocks over all m-blocks: each XCD's L2 holds its own
// slice of the weight.  Operand lane l: row l % 32 of the 32-row tile, codes
// of half l / 32 of the block (A and B split the block's 32 k-values alike,
// so the int32 dot is exact).  Accumulator layout: lane l holds column
// l % 32, register i holds row 8 * (i / 4) + 4 * (l / 32) + i % 4.  Tiles
// past the matrix (a last block of one 32-row tile) read the last tile again
// and are not stored.
// ONE: every wave has exactly one group (S = number of groups): no running
// sum across rounds, wave 0 sums into its own accumulators (y = 0 + a_0,
// then + a_1, ...).
template <int S, int TM, int TN, bool ONE>
__global__ __launch_bounds__(64 * S) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm(GemmArgs g) {
    extern __shared__ float4 part[];  // [S - 1][TM * TN][4][64]
    constexpr int T = TM * TN;
    const int lane = threadIdx.x & 63;
    const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ntm = g.ntm, ntn = (g.n + 31) / 32;
    const int nbm = (ntm + TM - 1) / TM;  // m-blocks of TM tiles
    const int wgi = blockIdx.x, per = g.ntiles >> 3, rem = g.ntiles & 7, xcd = wgi & 7, j8 = wgi >> 3;
    const int tl = xcd < rem ? xcd * (per + 1) + j8 : rem * (per + 1) + (xcd - rem) * per + j8;
    const int bn = tl / nbm, bm = tl - bn * nbm;
    const int half = lane >> 5, r32 = lane & 31;
    const bool lo = lane < 32;
    const int nb = g.nb, G = g.groups;
    GemmSrc<TM, TN> o;
    o.ra = __builtin_amdgcn_make_buffer_rsrc((void*)g.xq, (short)0, g.xq_bytes, RSRC_CFG);
    o.rb = __builtin_amdgcn_make_buffer_rsrc((void*)g.wc, (short)0, g.wc_bytes, RSRC_CFG);
    o.rx = __builtin_amdgcn_make_buffer_rsrc((void*)g.xs, (short)0, g.xs_bytes, RSRC_CFG);
    o.rw = __builtin_amdgcn_make_buffer_rsrc((void*)g.ws, (short)0, g.ws_bytes, RSRC_CFG);
    int mts[TM], nts[TN];
#pragma unroll
    for (int t = 0; t < TM; t++) {
        mts[t] = min(bm * TM + t, ntm - 1);
        o.oa[t] = ((mts[t] * 2 + (r32 >> 4)) * g.np * 64 + half * 16 + (r32 & 15)) * 16;
        o.ox[t] = (mts[t] * 2 * G * 64 + lane) * 16;
    }
#pragma unroll
    for (int t = 0; t < TN; t++) {
        nts[t] = min(bn * TN + t, ntn - 1);
        o.ob[t] = ((nts[t] * 2 + (r32 >> 4)) * g.np * 64 + half * 16 + (r32 & 15)) * 16;
        o.ow[t] = ((nts[t] * 2 + (r32 >> 4)) * 2 * g.np * 16 + (r32 & 15)) * 2;
    }

    float acc[T][16];
    float y[ONE ? 1 : T][16];  // the running sum over rounds (ONE: acc itself)
    float (*yy)[16] = ONE ? acc : y;
    if (!ONE) {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) yy[t][r] = 0.0f;
    }
    Quad<TM, TN> q0, q1;
    const int R = ONE ? 1 : (G + S - 1) / S;
    {
        const int g0 = min(s, G - 1);
        gemm_load(o, g0 * GEMM_GROUP, nb, q0);
        gemm_load(o, g0 * GEMM_GROUP + 4, nb, q1);
    }
    for (int j = 0; j + 1 < R; j++) {
        gemm_group<true>(o, j * S + s, min((j + 1) * S + s, G - 1), nb, lo, q0, q1, acc);
        gemm_combine<S, T, false>(part, j, s, lane, G, acc, yy);
    }
    if (s == 0 || (R - 1) * S + s < G) gemm_group<false>(o, (R - 1) * S + s, 0, nb, lo, q0, q1, acc);
    gemm_combine<S, T, ONE>(part, R - 1, s, lane, G, acc, yy);

    if (s != 0) return;
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int col = nts[tn] * 32 + r32;
        if (bn * TN + tn >= ntn || col >= g.n) continue;
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
            if (bm * TM + tm >= ntm) continue;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int row = mts[tm] * 32 + 8 * (i >> 2) + 4 * half + (i & 3);
                if (row < g.m) {
                    const size_t off = (size_t)row * g.n + col;
                    float v = yy[tm * TN + tn][i];
                    if (g.resid) v = g.resid[off] + v;
                    g.y[off] = v;
                }
            }
        }
    }
}

// One round, every group its own wave (S = groups): a (32 TM) x 32 output
// block per workgroup; wave s runs group s over TM 32 x 32 MFMA tiles that
// share each weight fragment.  The operands of block i + 1 are issued behind
// the compute of block i (a one-block window: few registers, so many waves
// per SIMD hide the load latency; deeper windows and issuing the whole group
// up front measured slower).  Every wave writes its group sums to LDS and all
// waves then finish the outputs, one 64-lane output row slot per wave and
// round (consecutive lanes own consecutive columns, so the LDS reads and the
// stores are coalesced), each in group order: y = 0 + a_0, then + a_1, ...
// (the oracle's order), then y = resid + y.
template <int S, int TM>
__global__ __launch_bounds__(64 * S) __attribute__((amdgpu_waves_per_eu(3))) void k_gemm_one(GemmArgs g) {
    extern __shared__ float gpart[];  // [S][TM][16][64] floats, then [S][256] u16 (weight scales)
    const int lane = threadIdx.x & 63;
    const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ntmb = (g.ntm + TM - 1) / TM;
    const int wgi = blockIdx.x, per = g.ntiles >> 3, rem = g.ntiles & 7, xcd = wgi & 7, j8 = wgi >> 3;
    const int tl = xcd < rem ? xcd * (per + 1) + j8 : rem * (per + 1) + (xcd - rem) * per + j8;
    const int bn = tl / ntmb, bm = tl - bn * ntmb;
    const int half = lane >> 5, r32 = lane & 31;
    const bool lo = lane < 32;
    const int nb = g.nb, G = g.groups;
    const auto ra = __builtin_amdgcn_make_buffer_rsrc((void*)g.xq, (short)0, g.xq_bytes, RSRC_CFG);
    const auto rb = __builtin_amdgcn_make_buffer_rsrc((void*)g.wc, (short)0, g.wc_bytes, RSRC_CFG);
    const auto rx = __builtin_amdgcn_make_buffer_rsrc((void*)g.xs, (short)0, g.xs_bytes, RSRC_CFG);
    const auto rw = __builtin_amdgcn_make_buffer_rsrc((void*)g.ws, (short)0, g.ws_bytes, RSRC_CFG);
    int oa[TM], ox[TM], mts[TM];
#pragma unroll
    for (int t = 0; t < TM; t++) {
        mts[t] = min(bm * TM + t, g.ntm - 1);
        oa[t] = ((mts[t] * 2 + (r32 >> 4)) * g.np * 64 + half * 16 + (r32 & 15)) * 16;
        ox[t] = (mts[t] * 2 * G * 64 + lane) * 16;
    }
    const int ob = ((bn * 2 + (r32 >> 4)) * g.np * 64 + half * 16 + (r32 & 15)) * 16;
    const int b0 = s * GEMM_GROUP;
    // the weight scales of the wave's 8 blocks for the block's 32 columns in
    // one 8-byte load per lane: the two 16-row tiles' scales of blocks
    // b0 .. b0 + 7 are 256 contiguous bytes each (lane l: tile 2 bn + l / 32,
    // block b0 + (l % 32) / 4, rows 4 (l % 4) .. + 3), staged in the wave's
    // LDS words [tile][block][16 rows] and read back per block (blocks past
    // nb read whatever lies there and get a zero scale below)
    uint16_t* wsl = (uint16_t*)(gpart + S * TM * 16 * 64) + s * 256;
    {
        const int off = ((bn * 2 + (lane >> 5)) * 2 * g.np + b0) * 32 + (lane & 31) * 8;
        *(uint2*)(wsl + lane * 4) = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, off, 0, 0));
    }
    v4i A[GEMM_GROUP][TM], B[GEMM_GROUP];
    v4i dx[2][TM];
    // operands of block i of the group (codes of blocks past nb are read from
    // block nb - 1 and cancelled by a zero scale below)
    auto load_block = [&](int i) {
        const int bc = min(b0 + i, nb - 1);
        const int cs = (bc >> 1) * 1024 + (bc & 1) * 512;
        if ((i & 3) == 0) {
#pragma unroll
            for (int t = 0; t < TM; t++)
                dx[i >> 2][t] = __builtin_bit_cast(
                    v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, ox[t], ((b0 >> 2) + (i >> 2)) * 1024, 0));
        }
#pragma unroll
        for (int t = 0; t < TM; t++)
            A[i][t] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, oa[t], cs, 0));
        B[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rb, ob, cs, 0));
    };
    const v16i zi = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const v16f zf = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    float acc[TM][16];
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[t][r] = 0.0f;
    load_block(0);
    __builtin_amdgcn_sched_barrier(0);
    // acc = fmaf((float)I_b, dw_b * dx_b, acc) per block in order (gemm_quad
    // explains the scale MFMA)
#pragma unroll
    for (int i = 0; i < GEMM_GROUP; i++) {
        const uint32_t dwi = wsl[(r32 >> 4) * 128 + i * 16 + (r32 & 15)];
        const uint2 bu = {(lo && b0 + i < nb) ? dwi : 0u, 0u};
#pragma unroll
        for (int t = 0; t < TM; t++) {
            const v16i I = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i][t], B[i], zi, 0, 0, 0);
            const uint2 au = {(uint32_t)dx[i >> 2][t][i & 3], 0u};
            const v16f P = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, au), __builtin_bit_cast(v4h, bu),
                                                                zf, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 16; r++) acc[t][r] = fmaf((float)I[r], P[r], acc[t][r]);
        }
        if (i + 1 < GEMM_GROUP) load_block(i + 1);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < TM; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) gpart[((s * TM + t) * 16 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    // output row slot q = (t, r) of the block per wave and round (wave-uniform),
    // column lane: wave s takes slots s, s + S, ...
    constexpr int NQ = TM * 16;
#pragma unroll
    for (int k = 0; k < (NQ + S - 1) / S; k++) {
        const int q = s + k * S;
        if (q < NQ) {
            const int r = q & 15, t = q >> 4;
            float y = 0.0f;
#pragma unroll
            for (int u = 0; u < S; u++) y = y + gpart[((u * TM + t) * 16 + r) * 64 + lane];
            const int row = mts[t] * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int col = bn * 32 + (lane & 31);
            if (bm * TM + t < g.ntm && row < g.m && col < g.n) {
                const size_t off = (size_t)row * g.n + col;
                if (g.resid) y = g.resid[off] + y;
                g.y[off] = y;
            }
        }
    }
}

// ---- small-M GEMM: 16 x 16 output tiles (v_mfma_i32_16x16x32_i8) -----------
//
// For few 32 x 32 tiles (M of a batch of sequences): one 16 (rows of x) x 16
// (rows of W) tile per workgroup, wave s runs group s (S = the number of
// groups, one round), the same per-block arithmetic and group order as
// k_gemm.  A 16-row tile chunk of pair p holds in lane (r, part) the codes
// 16 part .. 16 part + 15 of the pair (part 0, 1: block 2p; 2, 3: block
// 2p + 1); one permlane32 swap per dword turns it into the two blocks'
// operands (block 2p: lanes 0..31 their own low 8 bytes, lanes 32..63 the
// high 8 bytes of lane l - 32; block 2p + 1 the mirror image), so every lane
// group of 16 holds 8 codes of one block.  x and W are split alike, so the
// int32 dot of each block is exact.  Scale products: one
// v_mfma_f32_16x16x16f16 per block with dx (lanes 0..15, element 0) and dw
// (lanes 0..15 of a real block, element 0), zero elsewhere: D = dx * dw
// exactly, 0 past nb.  Accumulator: lane l holds column l % 16 of rows
// 4 (l / 16) .. 4 (l / 16) + 3.
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct Gemm16Args {
    const int8_t* xq;
    const uint32_t* xs;
    const int8_t* wc;
    const uint16_t* ws;
    float* y;
    const float* resid;
    int m, n, nb, np, nbp4, mt16, nt16;
    int xq_bytes, xs_bytes, wc_bytes, ws_bytes;
};

__device__ __forceinline__ void split_pair(const v4i c, long& b0, long& b1) {
    const auto p0 = __builtin_amdgcn_permlane32_swap((uint32_t)c[0], (uint32_t)c[2], false, false);
    const auto p1 = __builtin_amdgcn_permlane32_swap((uint32_t)c[1], (uint32_t)c[3], false, false);
    b0 = (long)((uint64_t)p0[0] | ((uint64_t)p1[0] << 32));
    b1 = (long)((uint64_t)p0[1] | ((uint64_t)p1[1] << 32));
}

template <int S>
__global__ __launch_bounds__(64 * S) void k_gemm16(Gemm16Args g) {
    __shared__ v4f part[S > 1 ? S - 1 : 1][64];
    const int lane = threadIdx.x & 63;
    const int s = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // workgroups of one XCD (ids congruent mod 8) take a contiguous run of
    // tiles; the m-tiles of one n-tile are neighbours (their weight reads
    // meet in that XCD's L2)
    const int ntiles = g.mt16 * g.nt16;
    const int wgi = blockIdx.x, per = ntiles >> 3, rem = ntiles & 7, xcd = wgi & 7, j8 = wgi >> 3;
    const int tl = xcd < rem ? xcd * (per + 1) + j8 : rem * (per + 1) + (xcd - rem) * per + j8;
    const int nt = tl / g.mt16, mt = tl - nt * g.mt16;
    const int r = lane & 15;
    const bool lo = lane < 16;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)g.xq, (short)0, g.xq_bytes, RSRC_CFG);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)g.wc, (short)0, g.wc_bytes, RSRC_CFG);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)g.xs, (short)0, g.xs_bytes, RSRC_CFG);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)g.ws, (short)0, g.ws_bytes, RSRC_CFG);
    const int np = g.np, nb = g.nb;
    // operands of group s: pairs 4 s .. 4 s + 3 (clamped to the last pair;
    // their blocks are past nb and get zero scales)
    v4i ac[4], wcv[4];
    uint32_t dw[GEMM_GROUP];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int p = min(4 * s + j, np - 1);
        ac[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, ((mt * np + p) * 64 + lane) * 16, 0, 0));
        wcv[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rb, ((nt * np + p) * 64 + lane) * 16, 0, 0));
    }
    const int row = mt * 16 + r;  // activation row of lanes 0..15 (the operand holds every row of the tile)
    v4i dxq[2];
#pragma unroll
    for (int q = 0; q < 2; q++)
        dxq[q] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                             rx, (((row >> 5) * g.nbp4 + 2 * s + q) * 64 + (row & 31)) * 16, 0, 0));
#pragma unroll
    for (int i = 0; i < GEMM_GROUP; i++)
        dw[i] = __builtin_amdgcn_raw_buffer_load_b16(rw, ((nt * 2 * np + min(GEMM_GROUP * s + i, nb - 1)) * 16 + r) * 2, 0, 0);
    const v4i zi = {0, 0, 0, 0};
    const v4f zf = {0, 0, 0, 0};
    v4f acc = zf;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        long a2[2], w2[2];
        split_pair(ac[j], a2[0], a2[1]);
        split_pair(wcv[j], w2[0], w2[1]);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int i = 2 * j + h, b = GEMM_GROUP * s + i;
            const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(a2[h], w2[h], zi, 0, 0, 0);
            const uint2 au = {lo ? (uint32_t)dxq[i >> 2][i & 3] : 0u, 0u};
            const uint2 bu = {(lo && b < nb) ? dw[i] : 0u, 0u};
            const v4f P = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(v4h, au), __builtin_bit_cast(v4h, bu),
                                                                zf, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; v++) acc[v] = fmaf((float)I[v], P[v], acc[v]);
        }
    }
    // group order: y = 0 + a_0, then + a_1, ... (wave 0 sums the others' from LDS)
    if (S > 1) {
        if (s > 0) part[s - 1][lane] = acc;
        __syncthreads();
    }
    if (s != 0) return;
    v4f y;
#pragma unroll
    for (int v = 0; v < 4; v++) y[v] = 0.0f + acc[v];
#pragma unroll
    for (int u = 1; u < S; u++) {
        const v4f t = part[u - 1][lane];
#pragma unroll
        for (int v = 0; v < 4; v++) y[v] = y[v] + t[v];
    }
    const int col = nt * 16 + r;
    if (col >= g.n) return;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        const int m = mt * 16 + 4 * (lane >> 4) + v;
        if (m < g.m) {
            const size_t off = (size_t)m * g.n + col;
            g.y[off] = g.resid ? g.resid[off] + y[v] : y[v];
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
// [m/32][nbp/4][64][4] u32 with nbp = 8 * groups: 1 KiB per 32 rows and 4 blocks.
size_t act_scale_bytes(int m, int k) {
    const size_t groups = ((size_t)k / 32 + GEMM_GROUP - 1) / GEMM_GROUP;
    return (size_t)((m + 31) / 32) * 2 * groups * 1024;
}

lq8_status launch_quantize_act(hipStream_t s, const float* x, int m, int k, int8_t* codes, uint32_t* scales) {
    const int groups = (k / 32 + GEMM_GROUP - 1) / GEMM_GROUP;
    const size_t waves = (size_t)((m + 31) / 32) * 2 * (4 * groups);
    if (!waves) return LQ8_OK;
    // two waves per workgroup: at M = 512 the gate/up and down operands end
    // to end 12.20 -> 12.09 and 13.89 -> 13.41 us against four
    hipLaunchKernelGGL(k_quantize_act, dim3(grid1(waves, 2)), dim3(128), 0, s, x, m, k, (int)waves, 4 * groups,
                       codes, scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

bool rms_quantize_supported(int dim) { return dim > 0 && dim % 32 == 0 && dim <= 64 * 32; }

lq8_status launch_rms_quantize_act(hipStream_t s, const float* x, const float* w, int m, int dim, float eps,
                                   int8_t* codes, uint32_t* scales) {
    if (!rms_quantize_supported(dim)) return fail(LQ8_ERR_SHAPE_MISMATCH, "rms_quantize_act: unsupported dim");
    if (m <= 0) return LQ8_OK;
    const int nb = dim / 32, np = (nb + 1) / 2, nbp = GEMM_GROUP * ((nb + GEMM_GROUP - 1) / GEMM_GROUP);
    const unsigned grid = (unsigned)((m + 31) / 32 * 8);  // 4 padded rows per workgroup
    const int u = (dim + 63) / 64;
    if (u <= 4)
        hipLaunchKernelGGL(k_rms_quantize_act<4>, dim3(grid), dim3(256), 0, s, x, w, m, dim, eps, np, nbp, codes, scales);
    else if (u <= 8)
        hipLaunchKernelGGL(k_rms_quantize_act<8>, dim3(grid), dim3(256), 0, s, x, w, m, dim, eps, np, nbp, codes, scales);
    else if (u <= 16)
        hipLaunchKernelGGL(k_rms_quantize_act<16>, dim3(grid), dim3(256), 0, s, x, w, m, dim, eps, np, nbp, codes,
                           scales);
    else
        hipLaunchKernelGGL(k_rms_quantize_act<32>, dim3(grid), dim3(256), 0, s, x, w, m, dim, eps, np, nbp, codes,
                           scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

bool combine_rms_quant_supported(int K, int dim) {
    return K >= 1 && K <= CRQ_MAX_K && rms_quantize_supported(dim) && dim <= CRQ_MAX_DIM;
}

lq8_status launch_combine_rms_quant(hipStream_t s, const float* h2, const float* eo, const uint32_t* rids,
                                    const float* rw, int K, int m, int dim, const float* w, float eps, float* out,
                                    int8_t* codes, uint32_t* scales) {
    if (!combine_rms_quant_supported(K, dim)) return fail(LQ8_ERR_SHAPE_MISMATCH, "combine_rms_quant: unsupported shape");
    if (m <= 0) return LQ8_OK;
    const int nb = dim / 32, np = (nb + 1) / 2, nbp = GEMM_GROUP * ((nb + GEMM_GROUP - 1) / GEMM_GROUP);
    const unsigned grid = (unsigned)((m + 31) / 32 * 32);  // the padded rows
    hipLaunchKernelGGL(k_combine_rms_quant, dim3(grid), dim3(CRQ_THREADS), 0, s, h2, eo, rids, rw, K, m, dim, w, eps,
                       np, nbp, out, codes, scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_silu_quantize_act(hipStream_t s, const float* gu, int m, int inter, int8_t* codes,
                                    uint32_t* scales) {
    if (inter <= 0 || inter % 32) return fail(LQ8_ERR_SHAPE_MISMATCH, "silu_quantize_act: unsupported width");
    if (m <= 0) return LQ8_OK;
    const int nb = inter / 32, np = (nb + 1) / 2, groups = (nb + GEMM_GROUP - 1) / GEMM_GROUP;
    const size_t waves = (size_t)((m + 31) / 32 * 32) * groups;
    if (waves > (size_t)INT32_MAX) return fail(LQ8_ERR_SHAPE_MISMATCH, "silu_quantize_act: too many rows");
    hipLaunchKernelGGL(k_silu_quantize_act, dim3(grid1(waves, 4)), dim3(256), 0, s, gu, m, inter, (int)waves, groups,
                       np, codes, scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_attention_combine_quant(hipStream_t s, const float* part, size_t part_stride, const int* d_pos,
                                          int batch, int num_heads, int cmax, int8_t* codes, uint32_t* scales) {
    if (batch <= 0 || num_heads <= 0 || cmax <= 0) return LQ8_OK;
    const int nb = num_heads * 4, np = (nb + 1) / 2, groups = (nb + GEMM_GROUP - 1) / GEMM_GROUP;
    hipLaunchKernelGGL(k_attn_combine_quant, dim3((unsigned)num_heads, (unsigned)batch), dim3(128), 0, s, part,
                       part_stride, d_pos, num_heads, cmax, np, 2 * groups, codes, scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_unpack_act(hipStream_t s, const int8_t* codes, const uint32_t* scales, int m, int k,
                             uint8_t* blocks) {
    const int nb = k / 32, np = (nb + 1) / 2, groups = (nb + GEMM_GROUP - 1) / GEMM_GROUP;
    const size_t n = (size_t)m * nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_unpack_act, dim3(grid1(n, WG)), dim3(WG), 0, s, codes, scales, m, nb, np, 2 * groups, blocks);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_quantize_aos(hipStream_t s, const float* x, size_t nblocks, uint8_t* blocks) {
    if (!nblocks) return LQ8_OK;
    hipLaunchKernelGGL(k_quantize_aos, dim3(grid1(nblocks, WG)), dim3(WG), 0, s, x, nblocks, blocks);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

// The 16 x 16 kernel (one round, a wave per group) when 32 x 32 tiles would
// leave most CUs idle: a batch of up to 64 rows against fewer than 512 tiles
// (M = 32: the 2048 x 4096 projection 14.1 -> 6.3 us, 5120 x 2048 8.8 -> 6.5
// us per call inside the 48-layer MoE step).
static bool gemm16_pick(int m, int groups, size_t tiles32) { return groups <= 16 && m <= 64 && tiles32 < 512; }

lq8_status launch_gemm(hipStream_t s, const int8_t* xq, const uint32_t* xs, int m, const lq8_weight* w, float* y,
                       const float* resid) {
    const size_t k = w->k_in;
    const size_t xq_bytes = act_code_bytes(m, (int)k), xs_bytes = act_scale_bytes(m, (int)k);
    const size_t wc_bytes = w->tiles * w->np * CHUNK_BYTES, ws_bytes = w->tiles * 2 * w->np * TILE_ROWS * 2;
    const size_t lim = (size_t)INT32_MAX;
    if (xq_bytes > lim || xs_bytes > lim || wc_bytes > lim || ws_bytes > lim)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "gemm: operand larger than 2 GiB");
    GemmArgs g;
    g.xq = xq;
    g.xs = xs;
    g.wc = w->codes;
    g.ws = w->scales;
    g.y = y;
    g.resid = resid;
    g.m = m;
    g.n = (int)w->n_out;
    g.nb = (int)w->nb;
    g.np = (int)w->np;
    g.groups = (g.nb + GEMM_GROUP - 1) / GEMM_GROUP;
    g.ntm = (m + 31) / 32;
    g.xq_bytes = (int)xq_bytes;
    g.xs_bytes = (int)xs_bytes;
    g.wc_bytes = (int)wc_bytes;
    g.ws_bytes = (int)ws_bytes;
    // K split over S waves (one group per wave per round).  S: every group its
    // own wave (one round, no running sum: k_gemm_one) when the groups are
    // few (<= 4) or the waves that gives stay <= 8192; otherwise the fewest of
    // 2, 3, 4, 6, 8, 12, 16 that give >= 2048 waves (k_gemm, one 32 x 32 tile
    // per workgroup, running sum over rounds).  k_gemm_one gives each wave two
    // 32-row tiles sharing the weight fragment for long K (8 - 12 groups) when
    // that still leaves >= 3072 waves (M = 512 down 8.0 -> 7.0 us); with fewer
    // groups or waves the single tile measured faster (M = 512 gate/up 8.6
    // against 8.7 us; M = 128 - 256 by 1 - 2 us).
    const int ntn = (g.n + 31) / 32;
    const size_t tiles = (size_t)g.ntm * ntn;
    if (tiles > lim) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemm: too many tiles");
    g.ntiles = (int)tiles;
    if (gemm16_pick(m, g.groups, tiles)) {
        Gemm16Args h;
        h.xq = xq; h.xs = xs; h.wc = w->codes; h.ws = w->scales; h.y = y; h.resid = resid;
        h.m = m; h.n = g.n; h.nb = g.nb; h.np = g.np; h.nbp4 = 2 * g.groups;
        h.mt16 = (m + 15) / 16;
        h.nt16 = (g.n + 15) / 16;
        h.xq_bytes = g.xq_bytes; h.xs_bytes = g.xs_bytes; h.wc_bytes = g.wc_bytes; h.ws_bytes = g.ws_bytes;
        const dim3 grid16((unsigned)(h.mt16 * h.nt16));
#define LQ8_GEMM16_CASE(SS) \
    case SS: hipLaunchKernelGGL((k_gemm16<SS>), grid16, dim3(64 * SS), 0, s, h); break;
        switch (g.groups) {
            LQ8_GEMM16_CASE(1) LQ8_GEMM16_CASE(2) LQ8_GEMM16_CASE(3) LQ8_GEMM16_CASE(4) LQ8_GEMM16_CASE(5)
            LQ8_GEMM16_CASE(6) LQ8_GEMM16_CASE(7) LQ8_GEMM16_CASE(8) LQ8_GEMM16_CASE(9) LQ8_GEMM16_CASE(10)
            LQ8_GEMM16_CASE(11) LQ8_GEMM16_CASE(12) LQ8_GEMM16_CASE(13) LQ8_GEMM16_CASE(14) LQ8_GEMM16_CASE(15)
            LQ8_GEMM16_CASE(16)
            default: return fail(LQ8_ERR_DEVICE, "gemm: no 16 x 16 kernel for this split");
        }
#undef LQ8_GEMM16_CASE
        LQ8_HIP(hipGetLastError());
        return LQ8_OK;
    }
    int S;
    if (g.groups <= 16 && (g.groups <= 4 || tiles * g.groups <= 8192)) {
        S = g.groups;
    } else {
        static const int kS[] = {2, 3, 4, 6, 8, 12, 16};
        S = 16;
        for (int c : kS)
            if (tiles * c >= 2048) { S = c; break; }
        S = std::min(S, g.groups);
    }
    if (S == g.groups) {
        const size_t tiles2 = (size_t)((g.ntm + 1) / 2) * ntn;
        const bool two = g.ntm >= 2 && S >= 8 && S <= 12 && tiles2 * S >= 3072;
        if (two) g.ntiles = (int)tiles2;
        const size_t smem1 = (size_t)S * (two ? 2 : 1) * 16 * 64 * sizeof(float) + (size_t)S * 256 * sizeof(uint16_t);
        const dim3 grid1d((unsigned)g.ntiles);
#define LQ8_GEMM_ONE_CASE(SS)                                                                          \
    case SS:                                                                                           \
        if (two) hipLaunchKernelGGL((k_gemm_one<SS, 2>), grid1d, dim3(64 * SS), smem1, s, g);           \
        else hipLaunchKernelGGL((k_gemm_one<SS, 1>), grid1d, dim3(64 * SS), smem1, s, g);               \
        break;
        switch (S) {
            LQ8_GEMM_ONE_CASE(1) LQ8_GEMM_ONE_CASE(2) LQ8_GEMM_ONE_CASE(3) LQ8_GEMM_ONE_CASE(4)
            LQ8_GEMM_ONE_CASE(5) LQ8_GEMM_ONE_CASE(6) LQ8_GEMM_ONE_CASE(7) LQ8_GEMM_ONE_CASE(8)
            LQ8_GEMM_ONE_CASE(9) LQ8_GEMM_ONE_CASE(10) LQ8_GEMM_ONE_CASE(11) LQ8_GEMM_ONE_CASE(12)
            LQ8_GEMM_ONE_CASE(13) LQ8_GEMM_ONE_CASE(14) LQ8_GEMM_ONE_CASE(15) LQ8_GEMM_ONE_CASE(16)
            default: return fail(LQ8_ERR_DEVICE, "gemm: no kernel for this split");
        }
#undef LQ8_GEMM_ONE_CASE
        LQ8_HIP(hipGetLastError());
        return LQ8_OK;
    }
    const size_t smem = (size_t)(S - 1) * 4 * 64 * sizeof(float4);
    const dim3 grid((unsigned)g.ntiles);
#define LQ8_GEMM_CASE(SS)                                                                          \
    case SS: hipLaunchKernelGGL((k_gemm<SS, 1, 1, false>), grid, dim3(64 * SS), smem, s, g); break;
    switch (S) {
        LQ8_GEMM_CASE(2) LQ8_GEMM_CASE(3) LQ8_GEMM_CASE(4) LQ8_GEMM_CASE(6) LQ8_GEMM_CASE(8) LQ8_GEMM_CASE(12)
        LQ8_GEMM_CASE(16)
        default: return fail(LQ8_ERR_DEVICE, "gemm: no kernel for this split");
    }
#undef LQ8_GEMM_CASE
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_repack_aos(hipStream_t s, const uint8_t* aos, size_t n_rows, size_t row0, const lq8_weight* w,
                             RowRun rr) {
    const size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_repack_aos, dim3(grid1(n, WG)), dim3(WG), 0, s, aos, n_rows, w->nb, w->np, row0, rr,
                       w->codes, w->scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_unpack_aos(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint8_t* aos,
                             RowRun rr) {
    const size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_unpack_aos, dim3(grid1(n, WG)), dim3(WG), 0, s, w->codes, w->scales, row0, rr, n_rows,
                       w->nb, w->np, aos);
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

lq8_status launch_quantize_weight_bf16(hipStream_t s, const uint16_t* src, size_t n_rows, size_t row0,
                                       const lq8_weight* w) {
    const size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    hipLaunchKernelGGL(k_quantize_weight_bf16, dim3(grid1(n, WG)), dim3(WG), 0, s, src, n_rows, row0, w->nb, w->np,
                       w->codes, w->scales);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_random_weight(hipStream_t s, const lq8_weight* w, size_t row0, size_t n_rows, uint64_t seed,
                                uint64_t stream, float stddev, RowRun rr) {
    const size_t n = n_rows * w->nb;
    if (!n) return LQ8_OK;
    const uint64_t key = seed * 0x9E3779B97F4A7C15ull ^ (stream + 1) * 0xC2B2AE3D27D4EB4Full;
    hipLaunchKernelGGL(k_random_weight, dim3(grid1(n, WG)), dim3(WG), 0, s, n_rows, row0, rr, w->nb, w->np, key,
                       stddev, w->codes, w->scales);
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
