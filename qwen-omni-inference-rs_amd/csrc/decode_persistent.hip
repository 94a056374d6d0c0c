// decode_persistent.hip -- greedy batch-1 Qwen3 decode as one persistent,
// cooperatively launched kernel: every decode step of a generate() call --
// all layers, the lm_head and the greedy pick -- with no kernel boundary in
// between.
//
// Work of one step (position pos), per layer:
//   P1  RmsNorm(h) + q|k|v GEMV, one 16-row tile per item
//   P2  attention, one (kv head, 64-position segment) per item; the last of
//       a kv head's segment items to finish (an arrival counter) combines the
//       segments into the head group's attention output
//   P3  o GEMV on the attention output + residual -> h2, one tile per item
//   P4  RmsNorm(h2) + gate and up GEMV (tile i of each) -> silu(gate) * up
//   P5  down GEMV + residual -> h, the next layer's input
// then P6: final RmsNorm and the lm_head, one wave per 16-row tile, each
// workgroup keeping the greedy pick of its tiles; the next step starts with
// every workgroup reducing the workgroups' picks to the token.  Item i of a
// phase belongs to workgroup i % P every step, so the workgroup that appends
// a kv head's key and value to a segment is the one that reads them later.
//
// Hand-off between workgroups: every value passed on is one 8-byte word (f32
// bits, then the step's tag), stored and loaded with agent-scope atomics
// (written through to, and read from, the device-coherent level).  A reader
// polls until each word it needs carries its step's tag, so the data is its
// own flag.  Buffers are per layer; a buffer is written again only one step
// later, by a producer whose inputs depend on the outputs of every reader of
// the earlier value.  Tags grow across launches (the host keeps the count)
// and zeroed buffers carry tag 0, which no step uses.
//
// Weights do not depend on the step's data: a workgroup issues a phase's
// weight loads (into registers) before it waits for the phase's inputs, so
// the weight stream overlaps the hand-offs.
//
// The arithmetic of every step is that of the separate kernels (gemv.hip,
// model_kernels.hip): the GEMV block tree, the SUM64 RmsNorm and its bf16
// roundings, the segment attention and its combine, silu(gate) * up, the
// residual adds, the last-index greedy pick -- so tokens and logits equal
// the graph-replayed path's bit for bit.
//
// Waits are bounded: a word that does not arrive within SYNC_SPIN_LIMIT
// polls sets the abort flag; every workgroup polls that flag while it waits
// and leaves its loops, and the host reports LQ8_ERR_DEVICE.
#include <algorithm>

#include "attn_device.h"
#include "decode_persistent.h"
#include "gemv_device.h"
#include "grid_sync.h"
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

#ifdef LQ8_PERSIST_TRACE
// Phase timeline (built with -DLQ8_PERSIST_TRACE only): thread 0 of every
// workgroup stamps s_memrealtime (100 MHz) at the marks of the fourth step of
// each launch, for the first LQ8_PTRACE_LAYERS layers.
__device__ uint64_t g_ptrace[LQ8_PTRACE_WG * LQ8_PTRACE_LAYERS * LQ8_PTRACE_POINTS];
__device__ __forceinline__ void ptrace_mark(int w, int s, int l, int pt) {
    if (s == 3 && threadIdx.x == 0 && w < LQ8_PTRACE_WG && l < LQ8_PTRACE_LAYERS)
        g_ptrace[((size_t)w * LQ8_PTRACE_LAYERS + l) * LQ8_PTRACE_POINTS + pt] = __builtin_amdgcn_s_memrealtime();
}
#define PTRACE(pt) ptrace_mark(w, s, l, pt)
#else
#define PTRACE(pt) ((void)0)
#endif

constexpr int PT = PERSIST_THREADS;
constexpr int PW = PT / 64;    // waves per workgroup
// Largest GEMV inputs: hidden (q|k|v, gate/up, lm_head), the attention
// output (o) and the intermediate size (down).
constexpr int K_H_MAX = 1024, K_Q_MAX = 2048, K_I_MAX = 4096;
// groups of two block pairs a wave holds for one tile of input length k
constexpr int groups_per_wave(int k) { return ((k / 64 + 1) / 2 + PW - 1) / PW; }
constexpr int NG_H = groups_per_wave(K_H_MAX), NG_Q = groups_per_wave(K_Q_MAX), NG_I = groups_per_wave(K_I_MAX);
constexpr int SLOTS = 2 * NG_I;  // weight chunks a wave holds in registers
constexpr int LM_MAX_NP = 16;  // lm_head tiles held per wave: up to 16 block pairs (hidden <= 1024)
constexpr int GS_TILE = PW * NG_I * 16;  // group sums of one tile (floats)
constexpr int CNT_STRIDE = 16;  // u32 per arrival counter (one per 64 bytes)

// A value the compiler must treat as produced here: per-thread index math
// derived from it is recomputed in each loop iteration instead of being
// hoisted to the kernel entry and held (spilled) across the whole kernel.
__device__ __forceinline__ int opaque(int x) {
    asm volatile("" : "+v"(x));
    return x;
}
// The same for the (uniform) argument block: its fields are loaded again
// (scalar cache) where they are used instead of being held in registers.
__device__ __forceinline__ const PersistArgs* opaque_args(const PersistArgs* p) {
    asm volatile("" : "+s"(p));
    return p;
}

__device__ __forceinline__ void tput(uint64_t* p, float v, unsigned tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t traw(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tok_tag(uint64_t v, unsigned tag) { return (unsigned)(v >> 32) == tag; }

// The value of a tagged word once it carries `tag`, given its first load v.
// Gives up (0, *bad set) after the poll limit or when another workgroup has
// raised the abort flag.
__device__ __forceinline__ float twait(const uint64_t* p, uint64_t v, unsigned tag, unsigned* abort_flag,
                                    volatile int* bad) {
    unsigned spins = 0;
    while (!tok_tag(v, tag)) {
        if (*bad) return 0.0f;
        if ((++spins & 63) == 0 && sync_load(abort_flag) != 0) {
            *bad = 1;
            return 0.0f;
        }
        if (spins > SYNC_SPIN_LIMIT) {
            __hip_atomic_fetch_or(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *bad = 1;
            return 0.0f;
        }
        __builtin_amdgcn_s_sleep(1);
        v = traw(p);
    }
    return __uint_as_float((unsigned)v);
}

__device__ __forceinline__ float tget(const uint64_t* p, unsigned tag, unsigned* abort_flag, volatile int* bad) {
    const uint64_t v = traw(p);
    return tok_tag(v, tag) ? __uint_as_float((unsigned)v) : twait(p, v, tag, abort_flag, bad);
}

// dst[i] = src[i] for i < n (tagged words), 8 loads per thread in flight.
__device__ __forceinline__ void tfetch(const uint64_t* src, int n, unsigned tag, float* dst, unsigned* abort_flag,
                                       volatile int* bad) {
    for (int i0 = threadIdx.x; i0 < n; i0 += 8 * PT) {
        uint64_t v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = traw(src + min(i0 + u * PT, n - 1));
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * PT;
            if (i < n)
                dst[i] = tok_tag(v[u], tag) ? __uint_as_float((unsigned)v[u]) : twait(src + i, v[u], tag, abort_flag, bad);
        }
    }
}

// Element j of row `row` of a tiled Q8_0 weight, dequantized (exact).
__device__ __forceinline__ float q8_elem(const int8_t* codes, const uint16_t* scales, int np, int row, int j) {
    const int tile = row / TILE_ROWS, r = row % TILE_ROWS, b = j >> 5, hf = (j >> 4) & 1;
    const float d = f16_bits_to_f32(scales[scale_off(tile, np, b, r)]);
    return d * (float)codes[code_off(tile, np, b, hf, r) + (j & 15)];
}

// ---- GEMV of one 16-row tile by the whole workgroup ----------------------------
// The tile's np block pairs form G = ceil(np / 2) groups of two pairs; wave w
// takes groups w, w + PW, ... (at most NG of them: np <= 2 * PW * NG), with
// the chunk loads of its gi-th group held in slots S0 + 2 gi, S0 + 2 gi + 1.
// The group sums meet in the pairwise tree over the groups: together the
// block tree of the GEMV order (gemv_tiles), bit for bit.
struct WRegs {
    u32x4 c[SLOTS];
    uint16_t d[SLOTS];
};

template <int S0, int NG>
__device__ __forceinline__ void tile_load(const int8_t* codes, const uint16_t* scales, int np, int tile, WRegs& R) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = (np + 1) >> 1;
    const int r = lane & 15, bsel = (lane >> 4) >> 1;
    const int8_t* cb = codes + (size_t)tile * np * CHUNK_BYTES + lane * 16;
    const uint16_t* sb = scales + (size_t)tile * 2 * np * 16 + bsel * 16 + r;
    // groups are taken in pairs: a wave with an odd group count also loads
    // (a copy of) the tile's last group as its last pair's partner
    const int ngr = G > wave ? (G - wave + PW - 1) / PW : 0;
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        if (gi < ((ngr + 1) & ~1)) {
            const int g = min(wave + gi * PW, G - 1);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int p = min(2 * g + i, np - 1);
                R.c[S0 + 2 * gi + i] = __builtin_nontemporal_load((const u32x4*)(cb + (size_t)p * CHUNK_BYTES));
                R.d[S0 + 2 * gi + i] = sb[(size_t)p * 32];
            }
        }
    }
}

// The 16 codes of a chunk, unpacked only where they are used: the empty asm
// keeps the compiler from hoisting the byte unpacking of every prefetched
// chunk next to its load (which would hold 16 registers per chunk).
__device__ __forceinline__ float dot16_pinned(u32x4 c, const float* __restrict__ x) {
    asm volatile("" : "+v"(c.x), "+v"(c.y), "+v"(c.z), "+v"(c.w));
    return dot16(c, x);
}

// Four chunk dots at once: the GEMV's 16-term chains (each in its order,
// from +0, as dot16), interleaved so that the four dependency chains overlap
// -- with one wave per SIMD nothing else hides their latency.  The codes are
// pinned here (see dot16_pinned).
__device__ __forceinline__ void dot16x4_pinned(u32x4 c0, u32x4 c1, u32x4 c2, u32x4 c3, const float* x0,
                                               const float* x1, const float* x2, const float* x3, float* out) {
    asm volatile("" : "+v"(c0.x), "+v"(c0.y), "+v"(c0.z), "+v"(c0.w), "+v"(c1.x), "+v"(c1.y), "+v"(c1.z), "+v"(c1.w),
                      "+v"(c2.x), "+v"(c2.y), "+v"(c2.z), "+v"(c2.w), "+v"(c3.x), "+v"(c3.y), "+v"(c3.z), "+v"(c3.w));
    const uint32_t w[4][4] = {{c0.x, c0.y, c0.z, c0.w}, {c1.x, c1.y, c1.z, c1.w}, {c2.x, c2.y, c2.z, c2.w},
                              {c3.x, c3.y, c3.z, c3.w}};
    const float* x[4] = {x0, x1, x2, x3};
    float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 xv[4];
#pragma unroll
        for (int k = 0; k < 4; k++) xv[k] = *(const float4*)(x[k] + 4 * i);
#pragma unroll
        for (int k = 0; k < 4; k++) p[k] = fmaf((float)(int8_t)(w[k][i] & 0xFF), xv[k].x, p[k]);
#pragma unroll
        for (int k = 0; k < 4; k++) p[k] = fmaf((float)(int8_t)((w[k][i] >> 8) & 0xFF), xv[k].y, p[k]);
#pragma unroll
        for (int k = 0; k < 4; k++) p[k] = fmaf((float)(int8_t)((w[k][i] >> 16) & 0xFF), xv[k].z, p[k]);
#pragma unroll
        for (int k = 0; k < 4; k++) p[k] = fmaf((float)(int8_t)(w[k][i] >> 24), xv[k].w, p[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) out[k] = p[k];
}

// Group sums of the wave's groups into gs[g * 16 + row], two groups (four
// chunks) at a time.
template <int S0, int NG>
__device__ __forceinline__ void tile_dot(const WRegs& R, const float* xs, int np, int nb, float* gs) {
    static_assert(NG % 2 == 0, "groups are taken in pairs");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = (np + 1) >> 1;
    const int part = lane >> 4, bsel = part >> 1, half = part & 1;
    const int ngr = G > wave ? (G - wave + PW - 1) / PW : 0;  // the wave's groups
#pragma unroll
    for (int gi = 0; gi < NG; gi += 2) {
        if (gi < ngr) {
            const bool two = gi + 1 < ngr;  // else the partner is the copy tile_load took (result unused)
            const int g0 = wave + gi * PW, g1 = min(g0 + PW, G - 1);
            const int p[4] = {min(2 * g0, np - 1), min(2 * g0 + 1, np - 1), min(2 * g1, np - 1), min(2 * g1 + 1, np - 1)};
            constexpr int s0 = S0 + 0;
            float h[4];
            dot16x4_pinned(R.c[s0 + 2 * gi], R.c[s0 + 2 * gi + 1], R.c[s0 + 2 * gi + 2], R.c[s0 + 2 * gi + 3],
                           xs + (2 * p[0] + bsel) * 32 + half * 16, xs + (2 * p[1] + bsel) * 32 + half * 16,
                           xs + (2 * p[2] + bsel) * 32 + half * 16, xs + (2 * p[3] + bsel) * 32 + half * 16, h);
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const LanePair hh = lanes16(h[k]);
                const float vb = (hh.lo + hh.hi) * f16_bits_to_f32(R.d[s0 + 2 * gi + k]);
                const LanePair vv = lanes32(vb);
                v[k] = 2 * p[k] + 1 >= nb ? vv.lo : vv.lo + vv.hi;
            }
            const float vg0 = 2 * g0 + 1 < np ? v[0] + v[1] : v[0];
            const float vg1 = 2 * g1 + 1 < np ? v[2] + v[3] : v[2];
            if (lane < 16) {
                gs[g0 * 16 + lane] = vg0;
                if (two) gs[g1 * 16 + lane] = vg1;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Row `lane` (< 16) of the tile: the pairwise tree over the G group sums, in
// place in gs (column `lane` per row).  Called by a whole wave: the four
// 16-lane quarters take the disjoint pairs of a level in turn, so the level's
// additions are the same ones in the same places as one lane per row doing
// them in order.
__device__ __forceinline__ float tile_final(float* gs, int G) {
    const int lane = threadIdx.x & 63, col = lane & 15, q = lane >> 4;
    for (int s = 1; s < G; s *= 2) {
        for (int i = 2 * s * q; i + s < G; i += 8 * s) gs[i * 16 + col] = gs[i * 16 + col] + gs[(i + s) * 16 + col];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    return gs[col];
}

// RmsNorm (src/rms_norm.rs:143-176) of xs[0, k) in place, in the order of
// the GEMV's XS_RMSNORM staging: bf16 inputs; SUM64 of squares (wave 0);
// inv = 1 / sqrt(sum / k + eps); out = bf16((v * inv) * bf16(w)).
__device__ __forceinline__ void stage_rmsnorm(float* xs, int k, const float* w, float eps, float* red) {
    const int tid = threadIdx.x;
    for (int i = tid; i < k; i += PT) xs[i] = bf16_round(xs[i]);
    __syncthreads();
    if (tid < 64) {
        float acc = 0.0f;
        for (int i = tid; i < k; i += 64) acc = acc + xs[i] * xs[i];
        acc = wave_sum64(acc);
        if (tid == 0) red[0] = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)k) + eps));
    }
    __syncthreads();
    const float inv = red[0];
    for (int i = tid; i < k; i += PT) xs[i] = bf16_round((xs[i] * inv) * bf16_round(w[i]));
    __syncthreads();
}

// zero the padding block of an odd block count (xs[k, 64 np))
__device__ __forceinline__ void stage_pad(float* xs, int k, int np) {
    for (int i = k + threadIdx.x; i < np * 64; i += PT) xs[i] = 0.0f;
}

// The attention output of kv head g's query heads (g G .. g G + G - 1) from
// the partials (o_c[128], m_c, l_c) of its C segments, in segment order: per
// head the running max m and denominator den with the coefficients
// a_c = exp(m - m'), b_c = exp(m_c - m'), then per element
// num = num * a_c + b_c * o_c and out = num / den -- the combine that the
// separate kernels do in the o GEMV's input staging.  lds: 33 G floats.
// Not inlined: only one workgroup per kv head runs it, and its registers stay
// out of the attention phase's allocation.
__device__ __noinline__ void combine_group(const uint64_t* partb, uint64_t* out, int g, int C, int NH, int G,
                                              unsigned tag, float* lds, unsigned* abort_flag, volatile int* bad) {
    const int tid = threadIdx.x;
    float* mcl = lds;                  // [C][G][2]
    float* coef = mcl + 2 * 8 * G;     // [C][G][2]
    float* dens = coef + 2 * 8 * G;    // [G]
    for (int q = tid; q < C * G; q += PT) {
        const uint64_t* p = partb + ((size_t)(q / G) * NH + g * G + q % G) * ATT_PART_STRIDE;
        mcl[2 * q] = tget(p + 128, tag, abort_flag, bad);
        mcl[2 * q + 1] = tget(p + 129, tag, abort_flag, bad);
    }
    __syncthreads();
    if (tid < G) {
        float m = -__builtin_huge_valf(), den = 0.0f;
        for (int c = 0; c < C; c++) {
            const int q = c * G + tid;
            const float mc = mcl[2 * q], lc = mcl[2 * q + 1];
            const float mn = m > mc ? m : mc;
            const float ea = expf_cr(m - mn), eb = expf_cr(mc - mn);
            coef[2 * q] = ea;
            coef[2 * q + 1] = eb;
            den = den * ea + eb * lc;
            m = mn;
        }
        dens[tid] = den;
    }
    __syncthreads();
    for (int i = tid; i < G * 128; i += PT) {
        const int hh = i >> 7, d = i & 127;
        uint64_t ro[8];  // C <= 8: every segment's word in flight together
#pragma unroll
        for (int c = 0; c < 8; c++)
            ro[c] = traw(partb + ((size_t)min(c, C - 1) * NH + g * G + hh) * ATT_PART_STRIDE + d);
        float num = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            if (c < C) {
                const uint64_t* p = partb + ((size_t)c * NH + g * G + hh) * ATT_PART_STRIDE + d;
                const float o = tok_tag(ro[c], tag) ? __uint_as_float((unsigned)ro[c]) : twait(p, ro[c], tag, abort_flag, bad);
                num = num * coef[2 * (c * G + hh)] + coef[2 * (c * G + hh) + 1] * o;
            }
        }
        tput(out + i, __fdiv_rn(num, dens[hh]), tag);
    }
}

struct Dims {
    int H, I, NH, NKV, G, QD, KD, QKV, npH, nbH, GH, npQ, nbQ, GQ, npI, nbI, GI;  // G*: groups of two pairs
};

__device__ __forceinline__ Dims dims_of(const PersistArgs& a) {
    Dims d;
    d.H = a.H; d.I = a.I; d.NH = a.NH; d.NKV = a.NKV; d.G = a.NH / a.NKV;
    d.QD = a.NH * 128; d.KD = a.NKV * 128; d.QKV = d.QD + 2 * d.KD;
    d.nbH = a.H >> 5; d.npH = (d.nbH + 1) >> 1; d.GH = (d.npH + 1) >> 1;
    d.nbQ = d.QD >> 5; d.npQ = (d.nbQ + 1) >> 1; d.GQ = (d.npQ + 1) >> 1;
    d.nbI = a.I >> 5; d.npI = (d.nbI + 1) >> 1; d.GI = (d.npI + 1) >> 1;
    return d;
}

// Per-phase locals, recomputed where used (from the opaque argument block):
// the model's dimensions, the phase item counts, the per-layer strides and
// the LDS layout -- region A (the staged GEMV input, or the attention
// segment and then the combine's scratch), then the group sums and the
// RmsNorm reduction.
#define PHASE_LOCALS                                                                                        \
    const Dims D = dims_of(a);                                                                              \
    const int T1 = (D.QKV + 15) / 16, TH = (D.H + 15) / 16, TI = D.I / 16, T6 = (a.vocab + 15) / 16;         \
    const int items2 = D.NKV * a.cmax;                                                                      \
    const size_t kv_layer = (size_t)D.NKV * a.max_pos * 128;                                                \
    const size_t part_layer = (size_t)a.cmax * D.NH * ATT_PART_STRIDE;                                      \
    float* xs = sm;                                                                                         \
    float* gs = sm + a.region_a;    /* [2][GS_TILE] */                                                      \
    float* red = gs + 2 * GS_TILE;  /* [16] */                                                              \
    float* qs = sm;                 /* attention: [G][128] */                                               \
    float* kn = qs + D.G * 128;     /* [128] */                                                             \
    float* vn = kn + 128;           /* [128] */                                                             \
    float* sc = vn + 128;           /* [G][64] */                                                           \
    float* mlc = sc + D.G * ATT_SEG; /* [G][2] */                                                           \
    float* ks = sm + seg_ks_off(D.G); /* [64][KPAD], later the V rows [64][128] */                           \
    (void)T1; (void)TH; (void)TI; (void)T6; (void)items2; (void)kv_layer; (void)part_layer; (void)xs;      \
    (void)gs; (void)red; (void)qs; (void)kn; (void)vn; (void)sc; (void)mlc; (void)ks

__global__ __launch_bounds__(PT) void k_decode_persistent(const PersistArgs* __restrict__ pa) {
    extern __shared__ float sm[];
    __shared__ int bad_s;
    __shared__ int last_s;
    __shared__ float pick_v[PW];
    __shared__ int pick_i[PW];
    volatile int* bad = &bad_s;
    const PersistArgs& a = *opaque_args(pa);
    const int P = gridDim.x, w = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (tid == 0) bad_s = 0;
    __syncthreads();

    uint32_t tok = 0;
    for (int s = 0; s < a.steps; s++) {
        const unsigned tag = a.tag0 + (unsigned)s;
        const int pos = a.pos0 + s;
        // ---- the step's input token: the previous step's greedy pick (last
        // index on ties) over the workgroups' picks; the first step's from
        // the previous kernel
        if (s == 0) {
            tok = *a.d_tok;
        } else {
            float bv = -__builtin_huge_valf();
            int bi = -1;
            for (int q = tid; q < P; q += PT) {
                const float v = tget(a.argb + 2 * q, tag - 1, a.abort_flag, bad);
                const int j = (int)__float_as_uint(tget(a.argb + 2 * q + 1, tag - 1, a.abort_flag, bad));
                if (v > bv || (v == bv && j > bi)) { bv = v; bi = j; }
            }
            argmax_step<32>(bv, bi);
            argmax_step<16>(bv, bi);
            argmax_step<8>(bv, bi);
            argmax_step<4>(bv, bi);
            argmax_step<2>(bv, bi);
            argmax_step<1>(bv, bi);
            if (lane == 0) { pick_v[wave] = bv; pick_i[wave] = bi; }
            __syncthreads();
            if (*bad) goto done;
            bv = pick_v[0];
            bi = pick_i[0];
            for (int q = 1; q < PW; q++)
                if (pick_v[q] > bv || (pick_v[q] == bv && pick_i[q] > bi)) { bv = pick_v[q]; bi = pick_i[q]; }
            const uint32_t picked = (uint32_t)(bi < 0 ? 0 : bi);
            if (w == 0 && tid == 0) a.tokens_out[a.step0 + s - 1] = picked;
            tok = a.feed_first ? a.tokens_out[0] : picked;
            __syncthreads();  // pick_v / pick_i are read before the next step writes them
        }

        for (int l = 0; l < pa->L; l++) {
            const PersistArgs& a = *opaque_args(pa);
            const int tid = opaque((int)threadIdx.x), lane = tid & 63;
            PHASE_LOCALS;
            const PLayer Lw = a.layers[l];
            uint64_t* qkvb = a.qkvb + (size_t)l * D.QKV;
            uint64_t* partb = a.partb + (size_t)l * part_layer;
            uint64_t* attnb = a.attnb + (size_t)l * D.QD;
            unsigned* cntb = a.cntb + (size_t)l * D.NKV * CNT_STRIDE;
            uint64_t* h2b = a.h2b + (size_t)l * D.H;
            uint64_t* actb = a.actb + (size_t)l * D.I;
            uint64_t* hb = a.hb + (size_t)l * D.H;
            const uint64_t* hin = l > 0 ? a.hb + (size_t)(l - 1) * D.H : nullptr;  // layer input (else the embedding)
            float* Kl = a.kc + l * kv_layer;
            float* Vl = a.vc + l * kv_layer;

            // ---- P1: RmsNorm(h) + q|k|v tiles
            if (w < T1) {
                PTRACE(LQ8_PT_P1_START);
                WRegs R;
                tile_load<0, NG_H>(Lw.qkv_c, Lw.qkv_s, D.npH, w, R);
                if (hin) tfetch(hin, D.H, tag, xs, a.abort_flag, bad);
                else
                    for (int j = tid; j < D.H; j += PT) xs[j] = q8_elem(a.emb_c, a.emb_s, D.npH, (int)tok, j);
                stage_pad(xs, D.H, D.npH);
                __syncthreads();
                if (*bad) goto done;
                stage_rmsnorm(xs, D.H, Lw.in_norm, a.eps, red);
                PTRACE(LQ8_PT_P1_NORMED);
                for (int t = w; t < T1; t += P) {
                    if (t != w) tile_load<0, NG_H>(Lw.qkv_c, Lw.qkv_s, D.npH, t, R);
                    tile_dot<0, NG_H>(R, xs, D.npH, D.nbH, gs);
                    __syncthreads();
                    if (tid < 64) {
                        const float y = tile_final(gs, D.GH);
                        const int row = t * 16 + tid;
                        if (tid < 16 && row < D.QKV) tput(qkvb + row, y, tag);
                    }
                    __syncthreads();
                }
            }

            // ---- P2: attention per (kv head, segment)
            PTRACE(LQ8_PT_P2_START);
            {
                const int L1 = pos + 1, C = (L1 + ATT_SEG - 1) / ATT_SEG;
                for (int it = w; it < items2; it += P) {
                    const int g = it / a.cmax, c = it % a.cmax;
                    if (c >= C) continue;
                    const int js = c * ATT_SEG, nj = min(ATT_SEG, L1 - js);
                    const bool last = c == C - 1;
                    const int newrow = last ? pos - js : -1;
                    float* Kc = Kl + (size_t)g * a.max_pos * 128;
                    float* Vc = Vl + (size_t)g * a.max_pos * 128;
                    float4 kreg[ATT_SEG * 32 / PT], vreg[ATT_SEG * 32 / PT];
                    seg_load<PT, true>(Kc, Vc, js, nj, kreg, vreg);
                    const float* cs = a.cos_t + (size_t)pos * 64;
                    const float* sn = a.sin_t + (size_t)pos * 64;
                    for (int t = wave; t < D.G + 2; t += PW) {
                        if (t >= D.G && !last) continue;
                        const uint64_t* src = t < D.G ? qkvb + (g * D.G + t) * 128
                                                      : qkvb + D.QD + (t == D.G ? 0 : D.KD) + g * 128;
                        const uint64_t r0 = traw(src + lane), r1 = traw(src + lane + 64);
                        const float x0 = tok_tag(r0, tag) ? __uint_as_float((unsigned)r0)
                                                          : twait(src + lane, r0, tag, a.abort_flag, bad);
                        const float x1 = tok_tag(r1, tag) ? __uint_as_float((unsigned)r1)
                                                          : twait(src + lane + 64, r1, tag, a.abort_flag, bad);
                        if (t < D.G) {
                            head_norm_rope_vals(x0, x1, Lw.q_norm[lane], Lw.q_norm[lane + 64], cs, sn, a.eps,
                                                qs + t * 128);
                        } else if (t == D.G) {
                            head_norm_rope_vals(x0, x1, Lw.k_norm[lane], Lw.k_norm[lane + 64], cs, sn, a.eps, kn);
                            float* kr = Kc + (size_t)pos * 128;
                            kr[lane] = kn[lane];
                            kr[lane + 64] = kn[lane + 64];
                        } else {
                            vn[lane] = x0;
                            vn[lane + 64] = x1;
                            float* vr = Vc + (size_t)pos * 128;
                            vr[lane] = x0;
                            vr[lane + 64] = x1;
                        }
                    }
                    __syncthreads();
                    if (*bad) goto done;
                    PTRACE(LQ8_PT_P2_QKV_IN);
                    seg_scores<PT, true>(kreg, nj, newrow, kn, qs, D.G, a.scale, ks, sc, mlc);
                    __syncthreads();
                    PTRACE(LQ8_PT_P2_SCORES);
                    seg_stage_v<PT, true>(vreg, nj, newrow, vn, ks);
                    __syncthreads();
                    for (int t = tid; t < D.G * 128; t += PT) {
                        const int h = t >> 7, d = t & 127;
                        const float o = pv_chain(sc + h * ATT_SEG, ks, d, nj);
                        uint64_t* p = partb + ((size_t)c * D.NH + g * D.G + h) * ATT_PART_STRIDE;
                        tput(p + d, o, tag);
                        if (d == 0) {
                            tput(p + 128, mlc[2 * h], tag);
                            tput(p + 129, mlc[2 * h + 1], tag);
                        }
                    }
                    // every partial of the item is stored (write-through) before
                    // the item arrives at kv head g's counter; the C-th arrival
                    // resets the counter for the next step and combines
                    PTRACE(LQ8_PT_P2_PARTIALS);
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                    if (tid == 0) {
                        unsigned* cn = cntb + (size_t)g * CNT_STRIDE;
                        const bool lastc = sync_add(cn, 1u) + 1 == (unsigned)C;
                        if (lastc) {
                            sync_store(cn, 0u);
                            __builtin_amdgcn_s_waitcnt(0);  // the reset lands before the output is published
                        }
                        last_s = lastc ? 1 : 0;
                    }
                    __syncthreads();
                    if (last_s) combine_group(partb, attnb + (size_t)g * D.G * 128, g, C, D.NH, D.G, tag, sm,
                                              a.abort_flag, bad);
                    __syncthreads();
                }
            }

            // ---- P3: o tile on the attention output, + residual -> h2
            PTRACE(LQ8_PT_P3_START);
            for (int t = w; t < TH; t += P) {
                WRegs R;
                tile_load<0, NG_Q>(Lw.o_c, Lw.o_s, D.npQ, t, R);
                const int row = t * 16 + tid;
                uint64_t rres = 0;  // the residual word, loaded early
                if (tid < 16 && row < D.H && hin) rres = traw(hin + row);
                tfetch(attnb, D.QD, tag, xs, a.abort_flag, bad);
                stage_pad(xs, D.QD, D.npQ);
                __syncthreads();
                if (*bad) goto done;
                PTRACE(LQ8_PT_P3_STAGED);
                tile_dot<0, NG_Q>(R, xs, D.npQ, D.nbQ, gs);
                __syncthreads();
                if (tid < 64) {
                    const float acc = tile_final(gs, D.GQ);
                    if (tid < 16 && row < D.H) {
                        const float res = hin ? (tok_tag(rres, tag) ? __uint_as_float((unsigned)rres)
                                                                    : twait(hin + row, rres, tag, a.abort_flag, bad))
                                              : q8_elem(a.emb_c, a.emb_s, D.npH, (int)tok, row);
                        tput(h2b + row, res + acc, tag);
                    }
                }
                __syncthreads();
            }

            // ---- P4: RmsNorm(h2) + gate / up tile pair -> silu(gate) * up
            PTRACE(LQ8_PT_P4_START);
            for (int t = w; t < TI; t += P) {
                WRegs R;
                tile_load<0, NG_H>(Lw.gu_c, Lw.gu_s, D.npH, t, R);
                tile_load<2 * NG_H, NG_H>(Lw.gu_c, Lw.gu_s, D.npH, TI + t, R);
                tfetch(h2b, D.H, tag, xs, a.abort_flag, bad);
                stage_pad(xs, D.H, D.npH);
                __syncthreads();
                if (*bad) goto done;
                PTRACE(LQ8_PT_P4_STAGED);
                stage_rmsnorm(xs, D.H, Lw.post_norm, a.eps, red);
                tile_dot<0, NG_H>(R, xs, D.npH, D.nbH, gs);
                tile_dot<2 * NG_H, NG_H>(R, xs, D.npH, D.nbH, gs + GS_TILE);
                __syncthreads();
                if (tid < 64) {
                    const float g = tile_final(gs, D.GH), u = tile_final(gs + GS_TILE, D.GH);
                    if (tid < 16) tput(actb + t * 16 + tid, silu_mul(g, u), tag);
                }
                __syncthreads();
            }

            // ---- P5: down tile + residual -> h
            PTRACE(LQ8_PT_P5_START);
            for (int t = w; t < TH; t += P) {
                WRegs R;
                tile_load<0, NG_I>(Lw.dn_c, Lw.dn_s, D.npI, t, R);
                const int row = t * 16 + tid;
                uint64_t rres = 0;
                if (tid < 16 && row < D.H) rres = traw(h2b + row);
                tfetch(actb, D.I, tag, xs, a.abort_flag, bad);
                stage_pad(xs, D.I, D.npI);
                __syncthreads();
                if (*bad) goto done;
                PTRACE(LQ8_PT_P5_STAGED);
                tile_dot<0, NG_I>(R, xs, D.npI, D.nbI, gs);
                __syncthreads();
                if (tid < 64) {
                    const float acc = tile_final(gs, D.GI);
                    if (tid < 16 && row < D.H) {
                        const float res = tok_tag(rres, tag) ? __uint_as_float((unsigned)rres)
                                                             : twait(h2b + row, rres, tag, a.abort_flag, bad);
                        tput(hb + row, res + acc, tag);
                    }
                }
                __syncthreads();
                PTRACE(LQ8_PT_P5_DONE);
            }
        }

        // ---- P6: final RmsNorm, lm_head tiles (one wave each), greedy pick
        {
            [[maybe_unused]] const int l = 0;  // the P6 marks sit in layer 0's row
            PTRACE(LQ8_PT_P6_START);
            const PersistArgs& a = *opaque_args(pa);
            const int tid = opaque((int)threadIdx.x), lane = tid & 63;
            PHASE_LOCALS;
            const int t0 = w * PW + wave, tstride = P * PW;
            const int np = D.npH, nb = D.nbH;
            const int part = lane >> 4, bsel = part >> 1, half = part & 1, r = lane & 15;
            u32x4 cv[LM_MAX_NP];
            uint16_t dv[LM_MAX_NP];
            auto load_tile = [&](int t) {
                const int8_t* cb = a.emb_c + (size_t)t * np * CHUNK_BYTES + lane * 16;
                const uint16_t* sb = a.emb_s + (size_t)t * 2 * np * 16 + bsel * 16 + r;
#pragma unroll
                for (int p = 0; p < LM_MAX_NP; p++) {
                    if (p < np) {
                        cv[p] = __builtin_nontemporal_load((const u32x4*)(cb + (size_t)p * CHUNK_BYTES));
                        dv[p] = sb[(size_t)p * 32];
                    }
                }
            };
            if (t0 < T6) load_tile(t0);
            tfetch(a.hb + (size_t)(a.L - 1) * D.H, D.H, tag, xs, a.abort_flag, bad);
            stage_pad(xs, D.H, np);
            __syncthreads();
            if (*bad) goto done;
            stage_rmsnorm(xs, D.H, a.final_norm, a.eps, red);
            PTRACE(LQ8_PT_P6_NORMED);
            float bv = -__builtin_huge_valf();
            int bi = -1;
            for (int t = t0; t < T6; t += tstride) {
                float v[LM_MAX_NP];
#pragma unroll
                for (int p = 0; p < LM_MAX_NP; p++) {
                    if (p < np) {
                        const float h = dot16_pinned(cv[p], xs + (2 * p + bsel) * 32 + half * 16);
                        const LanePair hh = lanes16(h);
                        const float vb = (hh.lo + hh.hi) * f16_bits_to_f32(dv[p]);
                        const LanePair vv = lanes32(vb);
                        v[p] = 2 * p + 1 >= nb ? vv.lo : vv.lo + vv.hi;
                        if (p & 1) __builtin_amdgcn_sched_barrier(0);
                    }
                }
                if (t + tstride < T6) load_tile(t + tstride);  // the next tile while this one reduces
#pragma unroll
                for (int s2 = 1; s2 < LM_MAX_NP; s2 *= 2)
#pragma unroll
                    for (int i = 0; i + s2 < LM_MAX_NP; i += 2 * s2)
                        if (i + s2 < np) v[i] = v[i] + v[i + s2];
                const int row = t * 16 + r;
                const bool valid = lane < 16 && row < a.vocab;
                float tv = valid ? v[0] : -__builtin_huge_valf();
                int ti = valid ? row : -1;
                argmax_step<8>(tv, ti);
                argmax_step<4>(tv, ti);
                argmax_step<2>(tv, ti);
                argmax_step<1>(tv, ti);
                if (tv > bv || (tv == bv && ti > bi)) { bv = tv; bi = ti; }
            }
            // lanes 0..15 hold the wave's pick (rows of lanes 16..63 were invalid)
            if (lane == 0) { pick_v[wave] = bv; pick_i[wave] = bi; }
            __syncthreads();
            if (tid == 0) {
                float wv = pick_v[0];
                int wi = pick_i[0];
                for (int q = 1; q < PW; q++)
                    if (pick_v[q] > wv || (pick_v[q] == wv && pick_i[q] > wi)) { wv = pick_v[q]; wi = pick_i[q]; }
                tput(a.argb + 2 * w, wv, tag);
                tput(a.argb + 2 * w + 1, __uint_as_float((unsigned)wi), tag);
            }
            __syncthreads();
            PTRACE(LQ8_PT_P6_DONE);
        }
    }

    // the last step's token, and the decode state for the next call
    if (w == 0) {
        const unsigned tag = a.tag0 + (unsigned)a.steps - 1;
        float bv = -__builtin_huge_valf();
        int bi = -1;
        for (int q = tid; q < P; q += PT) {
            const float v = tget(a.argb + 2 * q, tag, a.abort_flag, bad);
            const int j = (int)__float_as_uint(tget(a.argb + 2 * q + 1, tag, a.abort_flag, bad));
            if (v > bv || (v == bv && j > bi)) { bv = v; bi = j; }
        }
        argmax_step<32>(bv, bi);
        argmax_step<16>(bv, bi);
        argmax_step<8>(bv, bi);
        argmax_step<4>(bv, bi);
        argmax_step<2>(bv, bi);
        argmax_step<1>(bv, bi);
        if (lane == 0) { pick_v[wave] = bv; pick_i[wave] = bi; }
        __syncthreads();
        if (tid == 0 && !*bad) {
            for (int q = 1; q < PW; q++)
                if (pick_v[q] > bv || (pick_v[q] == bv && pick_i[q] > bi)) { bv = pick_v[q]; bi = pick_i[q]; }
            const uint32_t picked = (uint32_t)(bi < 0 ? 0 : bi);
            a.tokens_out[a.step0 + a.steps - 1] = picked;
            *a.d_tok = picked;
            *a.d_pos = a.pos0 + a.steps;
            *a.d_step = a.step0 + a.steps;
        }
    }
done:
    return;
}

}  // namespace

bool persist_supported(const PersistShape& s, int num_cus) {
    if (s.head_dim != 128 || s.NKV <= 0 || s.NH % s.NKV) return false;
    const int G = s.NH / s.NKV;
    if (G > ATT_MAX_GROUP) return false;
    // GEMV inputs within the groups a wave holds for a tile (hidden <= 1024
    // also lets a wave hold a whole lm_head tile, 16 block pairs); the
    // combine: up to 8 segments
    if (s.H % 32 || s.H > K_H_MAX || s.I % 32 || s.I > K_I_MAX || s.NH * 128 > K_Q_MAX) return false;
    if (s.max_pos > 8 * ATT_SEG || num_cus <= 0) return false;
    return persist_smem_bytes(s) <= 64 * 1024;
}

size_t persist_xs_floats(const PersistShape& s) {
    const int k = std::max(s.H, std::max(s.NH * 128, s.I));
    return (size_t)((k + 63) / 64 * 64 + 64);
}

size_t persist_region_a(const PersistShape& s) {
    const int G = s.NH / s.NKV;
    const size_t a1 = persist_xs_floats(s);
    // the attention segment; the combine's scratch (33 G floats) reuses it
    const size_t a2 = std::max((size_t)seg_ks_off(G) + (size_t)ATT_SEG * KPAD, (size_t)33 * G);
    return (std::max(a1, a2) + 3) & ~(size_t)3;
}

size_t persist_smem_bytes(const PersistShape& s) { return (persist_region_a(s) + 2 * GS_TILE + 16) * sizeof(float); }

lq8_status launch_decode_persistent(hipStream_t st, const PersistArgs* d_args, int smem_bytes, int num_wg) {
    const PersistArgs* args = d_args;
    void* kargs[] = {&args};
    const size_t smem = (size_t)smem_bytes;
    hipError_t e = hipLaunchCooperativeKernel((const void*)k_decode_persistent, dim3((unsigned)num_wg), dim3(PT),
                                              kargs, smem, st);
    if (e == hipErrorCooperativeLaunchTooLarge)
        return fail(LQ8_ERR_DEVICE, "persistent decode: the grid cannot be co-resident");
    if (e != hipSuccess) return hip_fail(e, "persistent decode launch");
    return LQ8_OK;
}

}  // namespace lq8

using namespace lq8;

extern "C" lq8_status lq8_persist_trace(lq8_ctx* ctx, uint64_t* out, size_t count) {
    if (!registry_has(ctx)) return fail(LQ8_ERR_INVALID_ARG, "invalid context handle");
    if (!out || count != (size_t)LQ8_PTRACE_WG * LQ8_PTRACE_LAYERS * LQ8_PTRACE_POINTS)
        return fail(LQ8_ERR_INVALID_ARG, "trace buffer must hold LQ8_PTRACE_WG * LQ8_PTRACE_LAYERS * LQ8_PTRACE_POINTS words");
#ifdef LQ8_PERSIST_TRACE
    LQ8_HIP(hipSetDevice(ctx->device));
    LQ8_HIP(hipMemcpyFromSymbol(out, HIP_SYMBOL(lq8::g_ptrace), count * sizeof(uint64_t)));
    return LQ8_OK;
#else
    return fail(LQ8_ERR_INVALID_ARG, "library built without LQ8_PERSIST_TRACE (make trace)");
#endif
}
