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
//          kept (all when top_k = 0); e_j = exp(z_j - z_0);
//          prefix sums over the kept entries in chunks of 64: chunk totals
//          t_c sequential from 0, P_c = t_0 + ... + t_{c-1} sequential from 0,
//          C_j = P_c + (entries of j's chunk up to j, sequential from 0);
//          S = C_{K-1}; the nucleus ends at the first j with
//          C_j >= top_p * S (at K - 1 when top_p >= 1);
//          u = (SplitMix64(seed + step * 0x9E3779B97F4A7C15) >> 40) * 2^-24,
//          r = u * C_end; the token is the first j <= end with C_j > r (end
//          when rounding leaves none).
// The order comes from a stable LSD radix sort (4 passes of 8 bits) of the
// 32-bit keys ~order_bits(z) (ascending key = descending z) with the token
// index as payload, fed in index order when T > 0 (ties: first index first)
// and in reverse index order when T = 0 (ties: last index first).  Every
// pass is a per-tile digit histogram and a scatter that sums the histogram
// columns itself: no atomics in global memory and nothing to clear between
// calls, so the whole sampler can be replayed from a captured graph.
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

constexpr int CHUNK = 64;
constexpr int SORT_THREADS = 256, SORT_IPT = 8, SORT_TILE = SORT_THREADS * SORT_IPT, RADIX = 256;

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

// Digit counts of tile b -> hist[b][256].
template <int PASS>
__global__ __launch_bounds__(SORT_THREADS) void k_sort_hist(SortIn in, uint32_t* __restrict__ hist) {
    __shared__ uint32_t cnt[RADIX];
    const int t = threadIdx.x, b = blockIdx.x;
    cnt[t] = 0;
    uint32_t k[SORT_IPT], ix[SORT_IPT];
    load_tile<PASS>(in, b, k, ix);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SORT_IPT; j++)
        if (b * SORT_TILE + j * SORT_THREADS + t < in.V) atomicAdd(&cnt[(k[j] >> (8 * PASS)) & 255u], 1u);
    __syncthreads();
    hist[(size_t)b * RADIX + t] = cnt[t];
}

// Stable scatter of tile b: rank = keys of smaller digits everywhere + keys of
// this digit in earlier tiles + earlier keys of this digit in this tile
// (rounds of 256 in tile order; within a round, lane order from ballots).
template <int PASS>
__global__ __launch_bounds__(SORT_THREADS) void k_sort_scatter(SortIn in, int nb, const uint32_t* __restrict__ hist,
                                                              uint32_t* __restrict__ keys_out,
                                                              uint32_t* __restrict__ idx_out) {
    __shared__ uint32_t base[RADIX];
    __shared__ uint32_t wcnt[SORT_THREADS / 64][RADIX];
    __shared__ uint32_t wtot[SORT_THREADS / 64];
    const int t = threadIdx.x, b = blockIdx.x, w = t >> 6, lane = t & 63;
    uint32_t k[SORT_IPT], ix[SORT_IPT];
    load_tile<PASS>(in, b, k, ix);
    // digit t: count over all tiles and over the tiles before b
    uint32_t tot = 0, pre = 0;
    {
        int bb = 0;
        for (; bb + 8 <= nb; bb += 8) {
            uint32_t h[8];
#pragma unroll
            for (int u = 0; u < 8; u++) h[u] = hist[(size_t)(bb + u) * RADIX + t];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                tot += h[u];
                pre += bb + u < b ? h[u] : 0u;
            }
        }
        for (; bb < nb; bb++) {
            const uint32_t h = hist[(size_t)bb * RADIX + t];
            tot += h;
            pre += bb < b ? h : 0u;
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
    for (int q = 0; q < SORT_THREADS / 64; q++) wcnt[q][t] = 0;
    __syncthreads();
    uint32_t excl = inc - tot;
    for (int q = 0; q < w; q++) excl += wtot[q];
    base[t] = excl + pre;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SORT_IPT; j++) {
        const bool valid = b * SORT_TILE + j * SORT_THREADS + t < in.V;
        const uint32_t d = (k[j] >> (8 * PASS)) & 255u;
        unsigned long long m = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; bit++) {
            const bool on = (d >> bit) & 1u;
            const unsigned long long bb = __ballot(on);
            m &= on ? bb : ~bb;
        }
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (valid && rank == 0) wcnt[w][d] = (uint32_t)__popcll(m);
        __syncthreads();
        if (valid) {
            uint32_t pos = base[d] + rank;
            for (int q = 0; q < w; q++) pos += wcnt[q][d];
            if (pos < (uint32_t)in.V) {
                keys_out[pos] = k[j];
                idx_out[pos] = ix[j];
            }
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int q = 0; q < SORT_THREADS / 64; q++) {
            add += wcnt[q][t];
            wcnt[q][t] = 0;
        }
        base[t] += add;
        __syncthreads();
    }
}

__device__ __forceinline__ int kept(const SampleCfg* cfg, int V) { return cfg->top_k > 0 ? min(cfg->top_k, V) : V; }

// One thread per chunk of 64 kept entries: t_c.
__global__ __launch_bounds__(256) void k_sample_chunks(const uint32_t* __restrict__ sorted, int V,
                                                       const SampleCfg* cfg, float* __restrict__ tot) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (cfg->temperature <= 0.0f) return;
    const int K = kept(cfg, V);
    if (c * CHUNK >= K) return;
    const float z0 = key_value(sorted[0]);
    const int j1 = min(c * CHUNK + CHUNK, K);
    float t = 0.0f;
    for (int j = c * CHUNK; j < j1; j++) t = t + expf_cr(key_value(sorted[j]) - z0);
    tot[c] = t;
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// First j in chunk c (entries up to jlast) with P + C_j-in-chunk passing the
// test (>= thr when ge, > thr otherwise); -1 when none.  *cj: that C_j.
__device__ int chunk_search(const uint32_t* sorted, float z0, int c, int jlast, float P, float thr, bool ge,
                            float* cj) {
    float I = 0.0f;
    for (int j = c * CHUNK; j <= jlast; j++) {
        I = I + expf_cr(key_value(sorted[j]) - z0);
        const float C = P + I;
        if (ge ? C >= thr : C > thr) {
            *cj = C;
            return j;
        }
        *cj = C;
    }
    return -1;
}

// The pick (one thread): the token, then the step bookkeeping.
__global__ void k_sample_pick(const uint32_t* __restrict__ sorted, const uint32_t* __restrict__ sidx, int V,
                              const float* __restrict__ tot,
                              const SampleCfg* cfg, int* d_step, uint32_t* d_tok, uint32_t* tokens_out, int* d_pos,
                              uint32_t* counts_out) {
    if (threadIdx.x != 0) return;
    const int step = *d_step;
    uint32_t token;
    if (cfg->temperature <= 0.0f) {
        token = sidx[0];
    } else {
        const int K = kept(cfg, V), nch = (K + CHUNK - 1) / CHUNK;
        const float z0 = key_value(sorted[0]);
        float S = 0.0f;
        for (int c = 0; c < nch; c++) S = S + tot[c];
        int end = K - 1;
        float Cend = S;
        if (cfg->top_p < 1.0f) {
            const float thr = cfg->top_p * S;
            float P = 0.0f;
            int c = 0;
            while (c < nch - 1 && !(P + tot[c] >= thr)) {
                P = P + tot[c];
                c++;
            }
            const int j = chunk_search(sorted, z0, c, min(c * CHUNK + CHUNK, K) - 1, P, thr, true, &Cend);
            end = j >= 0 ? j : min(c * CHUNK + CHUNK, K) - 1;
        }
        const uint64_t h = splitmix64(cfg->seed + (uint64_t)(uint32_t)step * 0x9E3779B97F4A7C15ull);
        const float u = (float)(uint32_t)(h >> 40) * 5.9604644775390625e-8f;  // 2^-24
        const float r = u * Cend;
        const int ce = end / CHUNK;
        float P = 0.0f;
        int c = 0;
        while (c < ce && !(P + tot[c] > r)) {
            P = P + tot[c];
            c++;
        }
        float cj;
        const int j = chunk_search(sorted, z0, c, c < ce ? c * CHUNK + CHUNK - 1 : end, P, r, false, &cj);
        token = sidx[j >= 0 ? j : end];
    }
    *d_tok = token;
    if (tokens_out) tokens_out[step] = token;
    *d_step = step + 1;
    if (d_pos) *d_pos = *d_pos + 1;
    if (counts_out) counts_out[token] = counts_out[token] + 1u;
}

inline unsigned grid256(size_t n) { return (unsigned)((n + 255) / 256); }
inline size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

struct SampleWork {
    uint32_t *ka, *kb, *ia, *ib, *hist;
    float* tot;
};

int sort_tiles(int vocab) { return (vocab + SORT_TILE - 1) / SORT_TILE; }

size_t sample_chunk_count(int vocab) { return (size_t)(vocab + CHUNK - 1) / CHUNK; }

// ka | kb | ia | ib ([vocab] each) | hist [tiles][256] | chunk totals
size_t work_layout(int vocab, void* base, SampleWork* w) {
    const size_t v = up256((size_t)vocab * 4), h = up256((size_t)sort_tiles(vocab) * RADIX * 4);
    char* p = (char*)base;
    if (w) {
        w->ka = (uint32_t*)p;
        w->kb = (uint32_t*)(p + v);
        w->ia = (uint32_t*)(p + 2 * v);
        w->ib = (uint32_t*)(p + 3 * v);
        w->hist = (uint32_t*)(p + 4 * v);
        w->tot = (float*)(p + 4 * v + h);
    }
    return 4 * v + h + up256(sample_chunk_count(vocab) * 4);
}

template <int PASS>
lq8_status sort_pass(hipStream_t s, SortIn in, int nb, uint32_t* hist, uint32_t* keys_out, uint32_t* idx_out) {
    hipLaunchKernelGGL(k_sort_hist<PASS>, dim3(nb), dim3(SORT_THREADS), 0, s, in, hist);
    LQ8_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_sort_scatter<PASS>, dim3(nb), dim3(SORT_THREADS), 0, s, in, nb, (const uint32_t*)hist,
                       keys_out, idx_out);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

}  // namespace

size_t sample_work_bytes(int vocab) { return work_layout(vocab, nullptr, nullptr); }

lq8_status launch_sample(hipStream_t s, const SampleLaunch& a) {
    if (a.vocab <= 0) return fail(LQ8_ERR_INVALID_ARG, "sample: empty vocabulary");
    if (!a.work) return fail(LQ8_ERR_INVALID_ARG, "sample: no workspace");
    SampleWork w;
    work_layout(a.vocab, a.work, &w);
    const int nb = sort_tiles(a.vocab);
    SortIn in{a.logits, a.counts, a.cfg, nullptr, nullptr, a.vocab};
    lq8_status st;
    if ((st = sort_pass<0>(s, in, nb, w.hist, w.ka, w.ia))) return st;
    in.keys = w.ka;
    in.idx = w.ia;
    if ((st = sort_pass<1>(s, in, nb, w.hist, w.kb, w.ib))) return st;
    in.keys = w.kb;
    in.idx = w.ib;
    if ((st = sort_pass<2>(s, in, nb, w.hist, w.ka, w.ia))) return st;
    in.keys = w.ka;
    in.idx = w.ia;
    if ((st = sort_pass<3>(s, in, nb, w.hist, w.kb, w.ib))) return st;
    hipLaunchKernelGGL(k_sample_chunks, dim3(grid256(sample_chunk_count(a.vocab))), dim3(256), 0, s,
                       (const uint32_t*)w.kb, a.vocab, a.cfg, w.tot);
    LQ8_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_sample_pick, dim3(1), dim3(64), 0, s, (const uint32_t*)w.kb, (const uint32_t*)w.ib, a.vocab,
                       (const float*)w.tot, a.cfg, a.d_step, a.d_tok, a.tokens_out, a.d_pos, a.counts_out);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

}  // namespace lq8

namespace lq8 {

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

}  // namespace lq8

using namespace lq8;

extern "C" lq8_status lq8_sample_device(lq8_ctx* ctx, const float* d_logits, size_t vocab, const uint32_t* d_counts,
                                        const lq8_sampling* cfg, uint32_t step, uint32_t* d_token) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid or released context handle");
    if (!d_logits || !d_token) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (vocab == 0 || vocab > (size_t)INT32_MAX) return fail(LQ8_ERR_INVALID_ARG, "vocab out of range");
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
    if ((st = launch_sample(ctx->stream, a))) return st;
    LQ8_HIP(hipStreamSynchronize(ctx->stream));
    return LQ8_OK;
}
