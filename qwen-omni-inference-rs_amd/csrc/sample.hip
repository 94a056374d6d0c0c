// sample.hip -- next-token sampling on the device: repetition penalty,
// temperature, top-k, top-p and a counter-based RNG.
//
// The reference's samplers are argmax stubs (src/generate.rs:191-329); the
// sampling rule is fixed here (and restated by the CPU oracle):
//   x_i  = logits[i] with the repetition penalty applied once per earlier
//          occurrence of token i (src/generate.rs:353-380: x > 0 -> x / p,
//          x < 0 -> x * p, 0 unchanged; off when |p - 1| < 1e-6)
//   T = 0: greedy -- the largest x_i, the last index on ties (sample_greedy)
//   T > 0: z_i = x_i / T; entries ordered by z descending, ties by index
//          ascending (the reference's stable sort); the first K = top_k are
//          kept (all when top_k = 0); integer weights
//          w_j = floor(2^32 * exp(z_j - z_0)) (0 for NaN), so every sum below
//          is exact in 64 bits and independent of summation order;
//          C_j = w_0 + ... + w_j, S = C_{K-1};
//          top_p < 1: p24 = floor(top_p * 2^24), thr = ceil(S * p24 / 2^24),
//          the nucleus ends at the first j with C_j >= thr (K - 1 otherwise);
//          u24 = SplitMix64(seed + step * 0x9E3779B97F4A7C15) >> 40,
//          r = floor(C_end * u24 / 2^24) < C_end; the token is the first j
//          with C_j > r (the first entry when C_end = 0).
// The order comes from a stable LSD radix sort (4 passes of 8 bits) of the
// 32-bit keys ~order_bits(z) (ascending key = descending z) with the token
// index as payload, fed in index order when T > 0 (ties: first index first)
// and in reverse index order when T = 0 (ties: last index first).  Each pass
// is a per-tile digit count and a scatter in which every tile sums its digit's
// row of counts itself: no tile waits on another, no global atomics, and
// nothing is cleared by a memset between calls, so the whole sampler replays
// from a captured graph.
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

constexpr int SORT_THREADS = 256, SORT_IPT = 4, SORT_TILE = SORT_THREADS * SORT_IPT, RADIX = 256;
constexpr int PICK_THREADS = 1024, PICK_MAX_TILES = PICK_THREADS;
constexpr int PICK_PER = SORT_TILE / PICK_THREADS;  // sorted entries per pick thread in one tile (1 or 2)
static_assert(PICK_PER == 1 || PICK_PER == 2, "pick covers a tile with 1 or 2 entries per thread");
constexpr int MAX_VOCAB = PICK_MAX_TILES * SORT_TILE;
// top-k path: candidates by the top 12 bits of the key, at most TK_CAP of them
constexpr int TK_BINS = 4096, TK_CAP = 4096, TK_MAXK = PICK_THREADS;

__device__ __forceinline__ uint32_t order_bits(float z) {
    const uint32_t b = __float_as_uint(z);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float from_order_bits(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
// sorted key -> z
__device__ __forceinline__ float key_value(uint32_t key) { return from_order_bits(~key); }

__device__ __forceinline__ float penalized(float x, uint32_t count, float p) {
    if (fabsf(p - 1.0f) < 1e-6f) return x;
    for (uint32_t c = 0; c < count; c++) {
        if (x > 0.0f) x = __fdiv_rn(x, p);
        else if (x < 0.0f) x = x * p;
    }
    return x;
}

// floor(2^32 * exp(z - z0)); z <= z0 unless NaN, so the weight is <= 2^32.
__device__ __forceinline__ unsigned long long weight_of(float z, float z0) {
    const float e = expf_cr(z - z0);
    if (!(e > 0.0f)) return 0ull;
    return (unsigned long long)fminf(e * 4294967296.0f, 4294967296.0f);
}

__device__ __forceinline__ int kept(const SampleCfg* cfg, int V) { return cfg->top_k > 0 ? min(cfg->top_k, V) : V; }

// Sort input position p (< V): its token index and key.
__device__ __forceinline__ uint32_t input_key(const float* __restrict__ logits, const uint32_t* __restrict__ counts,
                                              const SampleCfg* cfg, int V, int p, uint32_t* idx) {
    const float T = cfg->temperature;
    const int i = T > 0.0f ? p : V - 1 - p;
    *idx = (uint32_t)i;
    const float x = penalized(logits[i], counts ? counts[i] : 0u, cfg->penalty);
    return ~order_bits(T > 0.0f ? __fdiv_rn(x, T) : x);
}

struct SortIn {
    const float* logits;
    const uint32_t* counts;
    const SampleCfg* cfg;
    const uint32_t* keys;  // pass > 0
    const uint32_t* idx;   // pass > 0
    int V;
    int nb;                // tiles
    int row;               // stride of a digit's row of tile counts (nb rounded up to 4)
};

template <int PASS>
__device__ __forceinline__ void load_tile(const SortIn& in, int b, uint32_t (&k)[SORT_IPT], uint32_t (&ix)[SORT_IPT]) {
#pragma unroll
    for (int j = 0; j < SORT_IPT; j++) {
        const int p = b * SORT_TILE + j * SORT_THREADS + (int)threadIdx.x;
        k[j] = 0;
        ix[j] = 0;
        if (p < in.V) {
            if constexpr (PASS == 0) k[j] = input_key(in.logits, in.counts, in.cfg, in.V, p, &ix[j]);
            else {
                k[j] = in.keys[p];
                ix[j] = in.idx[p];
            }
        }
    }
}

// Lanes of the wave holding the same digit d (among the valid lanes).
__device__ __forceinline__ unsigned long long same_digit_lanes(uint32_t d, bool valid) {
    unsigned long long m = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; bit++) {
        const bool on = (d >> bit) & 1u;
        const unsigned long long bb = __ballot(on);
        m &= on ? bb : ~bb;
    }
    return m;
}
__device__ __forceinline__ uint32_t lanes_below(unsigned long long m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Digit counts of tile b for pass PASS -> count plane PASS (a row of tile
// counts per digit; the row padding zeroed).  One LDS add per distinct digit
// of a wave: float keys concentrate on few values of their upper bytes.
template <int PASS>
__global__ __launch_bounds__(SORT_THREADS) void k_sort_hist(SortIn in, uint32_t* __restrict__ planes) {
    __shared__ uint32_t cnt[RADIX];
    const int t = threadIdx.x, b = blockIdx.x;
    cnt[t] = 0;
    uint32_t* plane = planes + (size_t)PASS * RADIX * in.row;
    if (b == 0)
        for (int q = in.nb; q < in.row; q++) plane[(size_t)t * in.row + q] = 0u;
    uint32_t k[SORT_IPT], ix[SORT_IPT];
    load_tile<PASS>(in, b, k, ix);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SORT_IPT; j++) {
        const bool valid = b * SORT_TILE + j * SORT_THREADS + t < in.V;
        const uint32_t d = (k[j] >> (8 * PASS)) & 255u;
        const unsigned long long m = same_digit_lanes(d, valid);
        if (valid && lanes_below(m) == 0) atomicAdd(&cnt[d], (uint32_t)__popcll(m));
    }
    __syncthreads();
    plane[(size_t)t * in.row + b] = cnt[t];
}

// Stable scatter of tile b: rank = keys of smaller digits everywhere + keys of
// this digit in earlier tiles + earlier keys of this digit in this tile
// (rounds of 256 in tile order; within a round, lane order from ballots).
// One barrier per round: the per-wave counts rotate over three buffers and
// the running digit bases over two, so a buffer is cleared or rewritten only
// after a barrier that follows its last reader.
template <int PASS>
__global__ __launch_bounds__(SORT_THREADS) void k_sort_scatter(SortIn in, const uint32_t* __restrict__ planes,
                                                              uint32_t* __restrict__ keys_out,
                                                              uint32_t* __restrict__ idx_out) {
    constexpr int W = SORT_THREADS / 64;
    __shared__ uint32_t base[2][RADIX];
    __shared__ uint32_t wcnt[3][W][RADIX];
    __shared__ uint32_t wtot[W];
    const int t = threadIdx.x, b = blockIdx.x, w = t >> 6, lane = t & 63;
    uint32_t k[SORT_IPT], ix[SORT_IPT];
    load_tile<PASS>(in, b, k, ix);
    // digit t: count over all tiles and over the tiles before b (one row)
    const uint4* rowp = (const uint4*)(planes + (size_t)PASS * RADIX * in.row + (size_t)t * in.row);
    uint32_t tot = 0, pre = 0;
    {
        const int n4 = in.row >> 2;
        int q = 0;
        for (; q + 8 <= n4; q += 8) {
            uint4 h[8];
#pragma unroll
            for (int u = 0; u < 8; u++) h[u] = rowp[q + u];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int b0 = 4 * (q + u);
                tot += h[u].x + h[u].y + h[u].z + h[u].w;
                pre += (b0 < b ? h[u].x : 0u) + (b0 + 1 < b ? h[u].y : 0u) + (b0 + 2 < b ? h[u].z : 0u) +
                       (b0 + 3 < b ? h[u].w : 0u);
            }
        }
        for (; q < n4; q++) {
            const uint4 h = rowp[q];
            const int b0 = 4 * q;
            tot += h.x + h.y + h.z + h.w;
            pre += (b0 < b ? h.x : 0u) + (b0 + 1 < b ? h.y : 0u) + (b0 + 2 < b ? h.z : 0u) + (b0 + 3 < b ? h.w : 0u);
        }
    }
    // exclusive scan of the digit totals over the block
    uint32_t inc = tot;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(inc, d, 64);
        if (lane >= d) inc += o;
    }
    if (lane == 63) wtot[w] = inc;
#pragma unroll
    for (int r = 0; r < 3; r++)
#pragma unroll
        for (int q = 0; q < W; q++) wcnt[r][q][t] = 0;
    __syncthreads();
    uint32_t excl = inc - tot;
    for (int q = 0; q < w; q++) excl += wtot[q];
    base[0][t] = excl + pre;
#pragma unroll
    for (int j = 0; j < SORT_IPT; j++) {
        const int cur = j % 3, nb2 = j & 1;
        const bool valid = b * SORT_TILE + j * SORT_THREADS + t < in.V;
        const uint32_t d = (k[j] >> (8 * PASS)) & 255u;
        const unsigned long long m = same_digit_lanes(d, valid);
        const uint32_t rank = lanes_below(m);
        if (valid && rank == 0) wcnt[cur][w][d] = (uint32_t)__popcll(m);
        __syncthreads();
        // buffer of round j - 1: read before this barrier, written next in round j + 2
#pragma unroll
        for (int q = 0; q < W; q++) wcnt[(j + 2) % 3][q][t] = 0;
        if (valid) {
            uint32_t pos = base[nb2][d] + rank;
            for (int q = 0; q < w; q++) pos += wcnt[cur][q][d];
            if (pos < (uint32_t)in.V) {
                keys_out[pos] = k[j];
                idx_out[pos] = ix[j];
            }
        }
        uint32_t add = 0;
#pragma unroll
        for (int q = 0; q < W; q++) add += wcnt[cur][q][t];
        base[nb2 ^ 1][t] = base[nb2][t] + add;
    }
}

// Exact 64-bit sum over the block (any order).
__device__ __forceinline__ unsigned long long block_sum_u64(unsigned long long v, unsigned long long* red) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    if (lane == 0) red[w] = v;
    __syncthreads();
    unsigned long long s = 0;
    for (int q = 0; q < (int)(blockDim.x >> 6); q++) s += red[q];
    return s;
}

// Weight sum of each tile of the sorted kept entries.
__global__ __launch_bounds__(SORT_THREADS) void k_sample_weights(const uint32_t* __restrict__ sorted, int V,
                                                                const SampleCfg* cfg,
                                                                unsigned long long* __restrict__ part) {
    __shared__ unsigned long long red[SORT_THREADS / 64];
    if (cfg->temperature <= 0.0f) return;
    const int K = kept(cfg, V), b = blockIdx.x;
    if (b * SORT_TILE >= K) return;
    const float z0 = key_value(sorted[0]);
    unsigned long long s = 0;
#pragma unroll
    for (int j = 0; j < SORT_IPT; j++) {
        const int p = b * SORT_TILE + j * SORT_THREADS + (int)threadIdx.x;
        if (p < K) s += weight_of(key_value(sorted[p]), z0);
    }
    s = block_sum_u64(s, red);
    if (threadIdx.x == 0) part[b] = s;
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// floor (or ceil) of a * b / 2^24 for a < 2^63, b <= 2^24 (exact).
__device__ __forceinline__ unsigned long long mul_shr24(unsigned long long a, unsigned long long b, bool round_up) {
    const unsigned long long lo = a * b, hi = __umul64hi(a, b);
    unsigned long long q = (hi << 40) | (lo >> 24);
    if (round_up && (lo & 0xFFFFFFull)) q++;
    return q;
}

// Inclusive scan over the threads of the pick block (exact).
__device__ __forceinline__ unsigned long long block_scan_u64(unsigned long long v, unsigned long long* wsum) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const unsigned long long o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    __syncthreads();
    if (lane == 63) wsum[w] = v;
    __syncthreads();
    for (int q = 0; q < w; q++) v += wsum[q];
    return v;
}

struct PickShared {
    unsigned long long pre[PICK_MAX_TILES];  // inclusive prefix of the tile weights
    unsigned long long wsum[PICK_THREADS / 64];
    unsigned long long c_hit;
    uint32_t first_tile, first_j;
};

// The first tile whose inclusive prefix passes the test (>= thr when ge,
// > thr otherwise); nt when none.
__device__ int first_tile(PickShared& sh, int nt, unsigned long long thr, bool ge) {
    const int t = threadIdx.x;
    __syncthreads();
    if (t == 0) sh.first_tile = (uint32_t)nt;
    __syncthreads();
    if (t < nt && (ge ? sh.pre[t] >= thr : sh.pre[t] > thr)) atomicMin(&sh.first_tile, (uint32_t)t);
    __syncthreads();
    return (int)sh.first_tile;
}

// In tile tb (< nt): the first kept j with C_j passing the test, its C_j ->
// sh.c_hit; -1 when none.
__device__ int first_in_tile(PickShared& sh, const uint32_t* sorted, float z0, int K, int tb, unsigned long long thr,
                             bool ge) {
    const int t = threadIdx.x;
    const int p0 = tb * SORT_TILE + PICK_PER * t;
    const unsigned long long w0 = p0 < K ? weight_of(key_value(sorted[p0]), z0) : 0ull;
    const unsigned long long w1 = PICK_PER == 2 && p0 + 1 < K ? weight_of(key_value(sorted[p0 + 1]), z0) : 0ull;
    const unsigned long long before = tb > 0 ? sh.pre[tb - 1] : 0ull;
    const unsigned long long inc = block_scan_u64(w0 + w1, sh.wsum);
    const unsigned long long c0 = before + (inc - w1), c1 = before + inc;
    if (t == 0) sh.first_j = 0xFFFFFFFFu;
    __syncthreads();
    const bool h0 = p0 < K && (ge ? c0 >= thr : c0 > thr);
    const bool h1 = PICK_PER == 2 && p0 + 1 < K && (ge ? c1 >= thr : c1 > thr);
    if (h0 || h1) atomicMin(&sh.first_j, (uint32_t)(h0 ? p0 : p0 + 1));
    __syncthreads();
    const uint32_t j = sh.first_j;
    if (j == (uint32_t)p0) sh.c_hit = c0;
    if (PICK_PER == 2 && j == (uint32_t)p0 + 1) sh.c_hit = c1;
    __syncthreads();
    return j == 0xFFFFFFFFu ? -1 : (int)j;
}

// The pick (one block): the token, then the step bookkeeping.
__global__ __launch_bounds__(PICK_THREADS) void k_sample_pick(const uint32_t* __restrict__ sorted,
                                                              const uint32_t* __restrict__ sidx, int V,
                                                              const unsigned long long* __restrict__ part,
                                                              const SampleCfg* cfg, int* d_step, uint32_t* d_tok,
                                                              uint32_t* tokens_out, int* d_pos, uint32_t* counts_out) {
    __shared__ PickShared sh;
    const int t = threadIdx.x;
    const int step = *d_step;
    uint32_t token = sidx[0];
    if (cfg->temperature > 0.0f) {
        const int K = kept(cfg, V), nt = (K + SORT_TILE - 1) / SORT_TILE;
        const float z0 = key_value(sorted[0]);
        sh.pre[t] = block_scan_u64(t < nt ? part[t] : 0ull, sh.wsum);
        __syncthreads();
        const unsigned long long S = sh.pre[nt - 1];
        unsigned long long c_end = S;
        if (cfg->top_p < 1.0f) {
            const unsigned long long p24 = (unsigned long long)(cfg->top_p * 16777216.0f);
            const unsigned long long thr = mul_shr24(S, p24, true);
            const int tb = first_tile(sh, nt, thr, true);
            if (tb < nt && first_in_tile(sh, sorted, z0, K, tb, thr, true) >= 0) c_end = sh.c_hit;
        }
        const uint64_t h = splitmix64(cfg->seed + (uint64_t)(uint32_t)step * 0x9E3779B97F4A7C15ull);
        const unsigned long long r = mul_shr24(c_end, h >> 40, false);
        if (c_end > 0) {
            const int tb = first_tile(sh, nt, r, false);
            if (tb < nt) {
                const int j = first_in_tile(sh, sorted, z0, K, tb, r, false);
                if (j >= 0) token = sidx[j];
            }
        }
    }
    if (t != 0) return;
    *d_tok = token;
    if (tokens_out) tokens_out[step] = token;
    *d_step = step + 1;
    if (d_pos) *d_pos = *d_pos + 1;
    if (counts_out) counts_out[token] = counts_out[token] + 1u;
}

// ---- top-k path ----------------------------------------------------------
// The kept set of the rule is the K smallest 64-bit keys (key32 << 32 | index),
// key32 = ~order_bits(z).  With a histogram of key32's top 12 bits the bucket
// holding the K-th key is known; the keys of that bucket and of every smaller
// one are the candidates (usually a few hundred), gathered and sorted in one
// workgroup's LDS.  When they exceed TK_CAP, the pick selects the K keys
// exactly with three more histogram levels over all keys and a scan in index
// order for ties -- slower, same result.

// Keys in index order (T > 0) and the bucket counts of their top 12 bits.
__global__ __launch_bounds__(SORT_THREADS) void k_topk_hist(SortIn in, uint32_t* __restrict__ keys32,
                                                           uint32_t* __restrict__ ghist) {
    __shared__ uint32_t h[TK_BINS];
    const int t = threadIdx.x, b = blockIdx.x;
    for (int i = t; i < TK_BINS; i += SORT_THREADS) h[i] = 0u;
    uint32_t k[SORT_IPT], ix[SORT_IPT];
    load_tile<0>(in, b, k, ix);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SORT_IPT; j++) {
        const int p = b * SORT_TILE + j * SORT_THREADS + t;
        if (p < in.V) {
            keys32[p] = k[j];
            atomicAdd(&h[k[j] >> 20], 1u);
        }
    }
    __syncthreads();
    for (int i = t; i < TK_BINS; i += SORT_THREADS)
        if (h[i]) atomicAdd(&ghist[i], h[i]);
}

// Block-wide: the smallest bin whose inclusive prefix count reaches `need`
// (bins [0, PER * blockDim)); *cum: that prefix.  `hist` may be global or
// LDS; sh: [blockDim / 64 + 2] scratch.  The bin is clamped into range (the
// callers' totals always reach `need`).
template <int PER>
__device__ void prefix_bin(const uint32_t* hist, uint32_t need, uint32_t* sh, int* bin, uint32_t* cum) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, nw = blockDim.x >> 6;
    const int nbins = PER * (int)blockDim.x;
    uint32_t v[PER];
    uint32_t mine = 0;
#pragma unroll
    for (int i = 0; i < PER; i++) {
        v[i] = hist[t * PER + i];
        mine += v[i];
    }
    uint32_t inc = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(inc, d, 64);
        if (lane >= d) inc += o;
    }
    __syncthreads();
    if (lane == 63) sh[w] = inc;
    __syncthreads();
    uint32_t run = inc - mine;
    for (int q = 0; q < w; q++) run += sh[q];
    if (t == 0) {
        sh[nw] = (uint32_t)(nbins - 1);
        sh[nw + 1] = 0u;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PER; i++) {
        if (run < need && run + v[i] >= need) {
            sh[nw] = (uint32_t)(t * PER + i);
            sh[nw + 1] = run + v[i];
        }
        run += v[i];
    }
    __syncthreads();
    *bin = min((int)sh[nw], nbins - 1);
    *cum = sh[nw + 1];
    __syncthreads();
}

// Candidates: every key whose top 12 bits are at most the boundary bucket's.
// Block 0 also leaves the boundary bucket and its prefix count in meta[0..1].
__global__ __launch_bounds__(SORT_THREADS) void k_topk_gather(SortIn in, const uint32_t* __restrict__ keys32,
                                                             const uint32_t* __restrict__ ghist,
                                                             uint32_t* __restrict__ counter, uint32_t* __restrict__ meta,
                                                             unsigned long long* __restrict__ cand) {
    __shared__ uint32_t sh[SORT_THREADS / 64 + 2];
    const int t = threadIdx.x, b = blockIdx.x, lane = t & 63;
    int beta;
    uint32_t cum;
    prefix_bin<TK_BINS / SORT_THREADS>(ghist, (uint32_t)kept(in.cfg, in.V), sh, &beta, &cum);
    if (b == 0 && t == 0) {
        meta[0] = (uint32_t)beta;
        meta[1] = cum;
    }
    if (cum > (uint32_t)TK_CAP) return;  // the pick selects exactly instead
#pragma unroll
    for (int j = 0; j < SORT_IPT; j++) {
        const int p = b * SORT_TILE + j * SORT_THREADS + t;
        const uint32_t key = p < in.V ? keys32[p] : 0xFFFFFFFFu;
        const bool take = p < in.V && (int)(key >> 20) <= beta;
        const unsigned long long m = __ballot(take);
        uint32_t base = 0;
        if (lane == 0 && m) base = atomicAdd(counter, (uint32_t)__popcll(m));
        base = __shfl(base, 0, 64);
        const uint32_t pos = base + lanes_below(m);
        if (take && pos < (uint32_t)TK_CAP) cand[pos] = ((unsigned long long)key << 32) | (uint32_t)p;
    }
}

// Exclusive count of `flag` over the threads before this one (block-wide);
// *total: the block's count.  sh: [blockDim / 64 + 1].
__device__ uint32_t block_excl_count(bool flag, uint32_t* sh, uint32_t* total) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, nw = blockDim.x >> 6;
    const unsigned long long m = __ballot(flag);
    __syncthreads();
    if (lane == 0) sh[w] = (uint32_t)__popcll(m);
    __syncthreads();
    uint32_t before = lanes_below(m), tot = 0;
    for (int q = 0; q < nw; q++) {
        if (q < w) before += sh[q];
        tot += sh[q];
    }
    *total = tot;
    return before;
}

// Bucket counts of (key >> shift) & mask over the keys whose key >> pshift
// equals prefix, all V keys read by the block (loads eight deep).
__device__ void refine_hist(const uint32_t* __restrict__ keys32, int V, int pshift, uint32_t prefix, int shift,
                            uint32_t mask, uint32_t* hist) {
    for (int i0 = threadIdx.x; i0 < V; i0 += 8 * PICK_THREADS) {
        uint32_t k[8];
#pragma unroll
        for (int u = 0; u < 8; u++) k[u] = keys32[min(i0 + u * PICK_THREADS, V - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (i0 + u * PICK_THREADS < V && (k[u] >> pshift) == prefix) atomicAdd(&hist[(k[u] >> shift) & mask], 1u);
    }
}

struct TopkShared {
    unsigned long long sb[TK_CAP];  // candidate keys, then the sorted kept set
    uint32_t hist[TK_BINS];
    unsigned long long wsum[PICK_THREADS / 64];
    uint32_t sh[PICK_THREADS / 64 + 2];
    unsigned long long c_hit;
    uint32_t first_j, n_taken;
};

// The kept set sorted, returned (its first K entries): the candidates when
// they fit, else the exact selection.  Up to 1024 entries: a rank sort (keys
// are distinct) into the histogram's space; more: bitonic in place.
__device__ const unsigned long long* topk_select(TopkShared& s, const uint32_t* __restrict__ keys32,
                                                 const uint32_t* __restrict__ ghist, const uint32_t* __restrict__ meta,
                                                 const unsigned long long* __restrict__ cand, int V, int K) {
    const int t = threadIdx.x;
    const int beta = min((int)meta[0], TK_BINS - 1);
    const uint32_t cum = meta[1];
    int n = (int)cum;
    if (cum <= (uint32_t)TK_CAP) {
        for (int i = t; i < n; i += PICK_THREADS) s.sb[i] = cand[i];
    } else {
        // level 2: bits 19..8 inside bucket beta
        const uint32_t need1 = (uint32_t)K - (cum - ghist[beta]);
        for (int i = t; i < TK_BINS; i += PICK_THREADS) s.hist[i] = 0u;
        __syncthreads();
        refine_hist(keys32, V, 20, (uint32_t)beta, 8, 0xFFFu, s.hist);
        __syncthreads();
        int b2;
        uint32_t c2;
        prefix_bin<TK_BINS / PICK_THREADS>(s.hist, need1, s.sh, &b2, &c2);
        const uint32_t need2 = need1 - (c2 - s.hist[b2]);
        const uint32_t p24 = ((uint32_t)beta << 12) | (uint32_t)b2;
        // level 3: bits 7..0 inside that bucket
        __syncthreads();
        for (int i = t; i < PICK_THREADS; i += PICK_THREADS) s.hist[i] = 0u;
        __syncthreads();
        refine_hist(keys32, V, 8, p24, 0, 0xFFu, s.hist);
        __syncthreads();
        int b3;
        uint32_t c3;
        prefix_bin<1>(s.hist, need2, s.sh, &b3, &c3);  // bins 256 .. 1023 stay zero
        const uint32_t need3 = need2 - (c3 - s.hist[b3]);
        const uint32_t v = (p24 << 8) | (uint32_t)b3;
        // every key below v, and the need3 lowest indices holding v
        if (t == 0) s.n_taken = 0u;
        uint32_t eq_seen = 0;
        for (int c0 = 0; c0 < V; c0 += PICK_THREADS) {
            const int i = c0 + t;
            const uint32_t key = i < V ? keys32[i] : 0xFFFFFFFFu;
            const bool less = i < V && key < v, eq = i < V && key == v;
            uint32_t eq_tot;
            const uint32_t eq_rank = block_excl_count(eq, s.sh, &eq_tot);
            if (less || (eq && eq_seen + eq_rank < need3)) {
                const uint32_t pos = atomicAdd(&s.n_taken, 1u);
                if (pos < (uint32_t)TK_CAP) s.sb[pos] = ((unsigned long long)key << 32) | (uint32_t)i;
            }
            eq_seen += eq_tot;
        }
        __syncthreads();
        n = (int)min(s.n_taken, (uint32_t)TK_CAP);
    }
    __syncthreads();
    if (n <= PICK_THREADS) {
        unsigned long long* out = (unsigned long long*)s.hist;
        const unsigned long long mine = t < n ? s.sb[t] : 0ull;
        uint32_t rank = 0;
        if (t < n)
            for (int j = 0; j < n; j++) rank += s.sb[j] < mine ? 1u : 0u;
        __syncthreads();
        if (t < n) out[rank] = mine;
        __syncthreads();
        return out;
    }
    // bitonic sort of sb[0, N), N the power of two >= n, padding at the top
    int N = 2;
    while (N < n) N <<= 1;
    for (int i = n + t; i < N; i += PICK_THREADS) s.sb[i] = ~0ull;
    __syncthreads();
    for (int kk = 2; kk <= N; kk <<= 1)
        for (int jj = kk >> 1; jj > 0; jj >>= 1) {
            for (int i = t; i < N; i += PICK_THREADS) {
                const int ixj = i ^ jj;
                if (ixj > i) {
                    const unsigned long long a = s.sb[i], c = s.sb[ixj];
                    if ((i & kk) == 0 ? a > c : a < c) {
                        s.sb[i] = c;
                        s.sb[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    return s.sb;
}

// The pick over the sorted kept set (K <= 1024 entries, one per thread), the
// step bookkeeping, and the histogram and counter cleared for the next call.
__global__ __launch_bounds__(PICK_THREADS) void k_topk_pick(const uint32_t* __restrict__ keys32,
                                                            uint32_t* __restrict__ ghist, uint32_t* __restrict__ counter,
                                                            const uint32_t* __restrict__ meta,
                                                            const unsigned long long* __restrict__ cand, int V,
                                                            const SampleCfg* cfg, int* d_step, uint32_t* d_tok,
                                                            uint32_t* tokens_out, int* d_pos, uint32_t* counts_out) {
    __shared__ TopkShared s;
    const int t = threadIdx.x;
    const int step = *d_step;
    const int K = kept(cfg, V);
    const unsigned long long* sorted = topk_select(s, keys32, ghist, meta, cand, V, K);
    const float z0 = key_value((uint32_t)(sorted[0] >> 32));
    const unsigned long long w = t < K ? weight_of(key_value((uint32_t)(sorted[t] >> 32)), z0) : 0ull;
    const unsigned long long C = block_scan_u64(w, s.wsum);
    if (t == K - 1) s.c_hit = C;
    __syncthreads();
    const unsigned long long S = s.c_hit;
    unsigned long long c_end = S;
    __syncthreads();
    if (cfg->top_p < 1.0f) {
        const unsigned long long p24 = (unsigned long long)(cfg->top_p * 16777216.0f);
        const unsigned long long thr = mul_shr24(S, p24, true);
        if (t == 0) s.first_j = 0xFFFFFFFFu;
        __syncthreads();
        if (t < K && C >= thr) atomicMin(&s.first_j, (uint32_t)t);
        __syncthreads();
        if ((uint32_t)t == s.first_j) s.c_hit = C;
        __syncthreads();
        if (s.first_j != 0xFFFFFFFFu) c_end = s.c_hit;
    }
    const uint64_t h = splitmix64(cfg->seed + (uint64_t)(uint32_t)step * 0x9E3779B97F4A7C15ull);
    const unsigned long long r = mul_shr24(c_end, h >> 40, false);
    __syncthreads();
    if (t == 0) s.first_j = 0xFFFFFFFFu;
    __syncthreads();
    if (c_end > 0 && t < K && C > r) atomicMin(&s.first_j, (uint32_t)t);
    __syncthreads();
    const uint32_t j = s.first_j;
    const uint32_t token = (uint32_t)sorted[j < (uint32_t)K ? j : 0u];
    for (int i = t; i < TK_BINS; i += PICK_THREADS) ghist[i] = 0u;
    if (t != 0) return;
    *counter = 0u;
    *d_tok = token;
    if (tokens_out) tokens_out[step] = token;
    *d_step = step + 1;
    if (d_pos) *d_pos = *d_pos + 1;
    if (counts_out) counts_out[token] = counts_out[token] + 1u;
}

inline size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

struct SampleWork {
    uint32_t *ghist, *counter, *meta;
    unsigned long long* cand;
    uint32_t *ka, *kb, *ia, *ib, *planes;
    unsigned long long* part;
};

int sort_tiles(int vocab) { return (vocab + SORT_TILE - 1) / SORT_TILE; }
int row_stride(int vocab) { return (sort_tiles(vocab) + 3) & ~3; }
constexpr size_t ZERO_BYTES = ((size_t)TK_BINS * 4 + 4 + 255) & ~(size_t)255;
constexpr size_t META_OFF = ZERO_BYTES;  // boundary bucket and prefix count, written by the gather

// top-k histogram | counter (zeroed region) | meta | candidates [TK_CAP] |
// ka | kb | ia | ib ([vocab] each) | count planes [4][256][row] | tile weights
size_t work_layout(int vocab, void* base, SampleWork* w) {
    const size_t z = ZERO_BYTES + 256, c = up256((size_t)TK_CAP * 8);
    const size_t v = up256((size_t)vocab * 4), h = up256((size_t)4 * RADIX * row_stride(vocab) * 4);
    char* p = (char*)base;
    if (w) {
        w->ghist = (uint32_t*)p;
        w->counter = (uint32_t*)(p + (size_t)TK_BINS * 4);
        w->meta = (uint32_t*)(p + META_OFF);
        w->cand = (unsigned long long*)(p + z);
        p += z + c;
        w->ka = (uint32_t*)p;
        w->kb = (uint32_t*)(p + v);
        w->ia = (uint32_t*)(p + 2 * v);
        w->ib = (uint32_t*)(p + 3 * v);
        w->planes = (uint32_t*)(p + 4 * v);
        w->part = (unsigned long long*)(p + 4 * v + h);
    }
    return z + c + 4 * v + h + up256((size_t)sort_tiles(vocab) * 8);
}

template <int PASS>
lq8_status sort_pass(hipStream_t s, SortIn in, uint32_t* planes, uint32_t* keys_out, uint32_t* idx_out) {
    hipLaunchKernelGGL(k_sort_hist<PASS>, dim3(in.nb), dim3(SORT_THREADS), 0, s, in, planes);
    LQ8_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_sort_scatter<PASS>, dim3(in.nb), dim3(SORT_THREADS), 0, s, in, (const uint32_t*)planes,
                       keys_out, idx_out);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

}  // namespace

size_t sample_work_bytes(int vocab) { return work_layout(vocab, nullptr, nullptr); }
size_t sample_work_zero_bytes(int) { return ZERO_BYTES; }
bool sample_topk_path(const SampleCfg& c) { return c.temperature > 0.0f && c.top_k >= 1 && c.top_k <= TK_MAXK; }

lq8_status launch_sample(hipStream_t s, const SampleLaunch& a) {
    if (a.vocab <= 0 || a.vocab > MAX_VOCAB) return fail(LQ8_ERR_INVALID_ARG, "sample: vocabulary outside 1 .. 2^20");
    if (!a.work) return fail(LQ8_ERR_INVALID_ARG, "sample: no workspace");
    SampleWork w;
    work_layout(a.vocab, a.work, &w);
    SortIn in{a.logits, a.counts, a.cfg, nullptr, nullptr, a.vocab, sort_tiles(a.vocab), row_stride(a.vocab)};
    if (a.topk) {
        hipLaunchKernelGGL(k_topk_hist, dim3(in.nb), dim3(SORT_THREADS), 0, s, in, w.ka, w.ghist);
        LQ8_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_topk_gather, dim3(in.nb), dim3(SORT_THREADS), 0, s, in, (const uint32_t*)w.ka,
                           (const uint32_t*)w.ghist, w.counter, w.meta, w.cand);
        LQ8_HIP(hipGetLastError());
        hipLaunchKernelGGL(k_topk_pick, dim3(1), dim3(PICK_THREADS), 0, s, (const uint32_t*)w.ka, w.ghist, w.counter,
                           (const uint32_t*)w.meta, (const unsigned long long*)w.cand, a.vocab, a.cfg, a.d_step, a.d_tok, a.tokens_out, a.d_pos,
                           a.counts_out);
        LQ8_HIP(hipGetLastError());
        return LQ8_OK;
    }
    lq8_status st;
    if ((st = sort_pass<0>(s, in, w.planes, w.ka, w.ia))) return st;
    in.keys = w.ka;
    in.idx = w.ia;
    if ((st = sort_pass<1>(s, in, w.planes, w.kb, w.ib))) return st;
    in.keys = w.kb;
    in.idx = w.ib;
    if ((st = sort_pass<2>(s, in, w.planes, w.ka, w.ia))) return st;
    in.keys = w.ka;
    in.idx = w.ia;
    if ((st = sort_pass<3>(s, in, w.planes, w.kb, w.ib))) return st;
    hipLaunchKernelGGL(k_sample_weights, dim3(in.nb), dim3(SORT_THREADS), 0, s, (const uint32_t*)w.kb, a.vocab, a.cfg,
                       w.part);
    LQ8_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_sample_pick, dim3(1), dim3(PICK_THREADS), 0, s, (const uint32_t*)w.kb, (const uint32_t*)w.ib,
                       a.vocab, (const unsigned long long*)w.part, a.cfg, a.d_step, a.d_tok, a.tokens_out, a.d_pos,
                       a.counts_out);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status check_sampling(const lq8_sampling* c, SampleCfg* out) {
    if (!c) return fail(LQ8_ERR_INVALID_ARG, "sampling config is null");
    // GenerationConfig::new (src/generate.rs:96-128)
    if (!(c->temperature >= 0.0f)) return fail(LQ8_ERR_INVALID_ARG, "temperature must be >= 0.0");
    if (!(c->top_p >= 0.0f && c->top_p <= 1.0f)) return fail(LQ8_ERR_INVALID_ARG, "top_p must be in [0.0, 1.0]");
    if (!(c->repetition_penalty >= 1.0f)) return fail(LQ8_ERR_INVALID_ARG, "repetition_penalty must be >= 1.0");
    if (c->top_k > (uint32_t)INT32_MAX) return fail(LQ8_ERR_INVALID_ARG, "top_k too large");
    out->temperature = c->temperature;
    out->top_k = (int)c->top_k;
    out->top_p = c->top_p;
    out->penalty = c->repetition_penalty;
    out->seed = c->seed;
    return LQ8_OK;
}

bool sample_vocab_ok(size_t vocab) { return vocab >= 1 && vocab <= (size_t)MAX_VOCAB; }

}  // namespace lq8

using namespace lq8;

extern "C" lq8_status lq8_sample_device(lq8_ctx* ctx, const float* d_logits, size_t vocab, const uint32_t* d_counts,
                                        const lq8_sampling* cfg, uint32_t step, uint32_t* d_token) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid or released context handle");
    if (!d_logits || !d_token) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (!sample_vocab_ok(vocab)) return fail(LQ8_ERR_INVALID_ARG, "vocab out of range (1 .. 2^20)");
    if (step > (uint32_t)INT32_MAX) return fail(LQ8_ERR_INVALID_ARG, "step out of range");
    SampleCfg sc;
    lq8_status st = check_sampling(cfg, &sc);
    if (st) return st;
    LQ8_HIP(hipSetDevice(ctx->device));
    const int V = (int)vocab;
    const size_t total = 256 + sample_work_bytes(V);
    void* scratch = nullptr;
    if ((st = ctx_scratch(ctx, total, &scratch))) return st;
    char* base = (char*)scratch;
    const int step_i = (int)step;
    LQ8_HIP(hipMemcpyAsync(base, &sc, sizeof(sc), hipMemcpyHostToDevice, ctx->stream));
    LQ8_HIP(hipMemcpyAsync(base + 64, &step_i, sizeof(int), hipMemcpyHostToDevice, ctx->stream));
    SampleLaunch a{};
    a.logits = d_logits;
    a.vocab = V;
    a.counts = d_counts;
    a.cfg = (const SampleCfg*)base;
    a.d_step = (int*)(base + 64);
    a.d_tok = d_token;
    a.work = base + 256;
    a.topk = sample_topk_path(sc);
    LQ8_HIP(hipMemsetAsync(a.work, 0, sample_work_zero_bytes(V), ctx->stream));
    if ((st = launch_sample(ctx->stream, a))) return st;
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    return LQ8_OK;
}
