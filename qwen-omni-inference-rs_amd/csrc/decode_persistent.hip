// decode_persistent.hip -- greedy batch-1 Qwen3 decode as one persistent,
// cooperatively launched kernel: every decode step of a generate() call --
// all layers, the lm_head and the greedy pick -- with no kernel boundary in
// between.  One workgroup of 512 threads (8 waves) per CU.
//
// Work of one step (position pos), per layer l (h_l the layer's input):
//   P1  h_l = h2 of layer l - 1 + its down projection's chunk sums (joined in
//       the GEMV block tree; published for P4), RmsNorm(h_l) + q|k|v GEMV,
//       one 16-row tile per item
//   P2  attention, one (64-position segment, kv head) per item: per query
//       head the segment's partials (o_c, m_c, l_c).  When a step has more
//       segments than one P3 gather holds (cdir), the item of the newest
//       segment keeps its own partials, reads the others' and combines the
//       kv head's segments (any number of them), publishing its heads'
//       attention output; a combiner waits only on items of lower index,
//       which every workgroup takes first, so the waits always end
//   P3  o GEMV, one (16-row tile, input chunk) per item: the chunk is csO
//       blocks of the attention output (whole heads or part of one), which
//       the item combines itself from the segment partials of its heads
//       (C <= cdir: one hand-off fewer than a separate combine) or fetches
//       from the combiners; the item's output is the tile's partial sum over
//       its chunk
//   P4  h2 = h_l + o (the chunk sums meet in the GEMV block tree), then
//       RmsNorm(h2) + gate and up GEMV (tile i of each) -> silu(gate) * up
//   P5  down GEMV, one (16-row tile, input chunk of csD block pairs) per
//       item: the tile's partial sum over its chunk (the residual h2 is
//       added where the chunk sums meet, in the next P1 or in P6)
// then P6: final RmsNorm and the lm_head, one wave per 16-row tile, each
// workgroup keeping the greedy pick of its tiles; the next step starts with
// every workgroup reducing the workgroups' picks to the token.  Item i of a
// phase belongs to workgroup i % P every step, so the workgroup that appends
// a kv head's key and value to a segment is the one that reads them later.
//
// Hand-off between workgroups: every value passed on is one 8-byte word (f32
// bits, then the step's tag), stored and loaded with agent-scope atomics
// (written through to, and read from, the device-coherent level).  A reader
// waits until each word it needs carries its step's tag, so the data is its
// own flag: all of a thread's words are loaded at once; while some are not
// there yet, one lane of the wave polls one of them and, when it lands, the
// wave loads its missing words again at once (so the polling traffic is one
// word per wave, and the fetch ends about one memory round trip after its
// last word lands).  Buffers are per layer; a buffer is written again only
// one step later, by a producer whose inputs depend on the outputs of every
// reader of the earlier value.  The greedy picks are the exception: every
// workgroup reads them, including workgroups that produce nothing else, so
// they alternate between two buffers by the parity of the step's tag (a
// workgroup cannot write step s + 2's pick before every workgroup has
// published step s + 1's, which each does after reading step s's).  Tags
// grow across launches (the host keeps the count) and zeroed buffers carry
// tag 0, which no step uses.
//
// Weights do not depend on the step's data: a workgroup issues the weight
// loads of its next phase's item (into registers) before it waits for the
// current phase's inputs, so the weight stream overlaps the hand-offs.
//
// The arithmetic of every step is that of the separate kernels (gemv.hip,
// model_kernels.hip): the GEMV block tree (an input chunk of a power-of-two
// block count aligned to its size is a subtree, and the chunk sums meet in
// the tree's upper levels), the SUM64 RmsNorm and its bf16 roundings, the
// segment attention and its combine, silu(gate) * up, the residual adds, the
// last-index greedy pick -- so tokens and logits equal the graph-replayed
// path's bit for bit.
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
constexpr int PW = PT / 64;     // waves per workgroup
// hand-off words per thread of each fetch (units t + u * PT)
constexpr int NW_ARG = (2 * 1024 + PT - 1) / PT;                   // the picks: 2 words per workgroup (<= 1024)
constexpr int NW_QKV = ((ATT_MAX_GROUP + 2) * 128 + PT - 1) / PT;  // q of a kv head's group, k, v
constexpr int NW_RES = PERSIST_FETCH;                             // h and the o chunk sums
// the instance for hidden above 1024 (HC = 4) gathers a hidden vector and
// its chunk sums in NW_RES4 words per thread and joins at most NCH4 chunk
// sums per element (fewer registers held across its phases)
constexpr int NW_RES4 = 12;
constexpr int NCH4 = 2;
template <int HC> constexpr int nw_res() { return HC == 4 ? NW_RES4 : NW_RES; }
template <int HC> constexpr int nch_max() { return HC == 4 ? NCH4 : PERSIST_NCH; }
constexpr int NW_ACT = (4096 + 16 + PT - 1) / PT;                  // silu(gate) * up (<= 4096) and 16 rows of h2
constexpr int NW_ATT = (2048 + PT - 1) / PT;                       // an o input chunk of the attention output (<= 2048)
constexpr int NW_PART = 16;                                        // an o chunk's segment partials ([C][R] words)
constexpr int CMB_SEGS = 64;                                       // combine: segments per batch, at most
constexpr int NW_ML = 1;                                           // combine: a batch's (m_c, l_c) words per thread
constexpr int CMB_EK = (ATT_MAX_GROUP * 128 + PT - 1) / PT;        // combine: output elements per thread, at most
constexpr int NW_OC = 16;                                          // combine: o_c words per thread and round
// HC (a kernel parameter, 2 or 4): block pairs per wave group of a
// hidden-long tile (q|k|v, gate/up, lm_head; K = hidden), so hidden <= 64 HC
// PW (1024 or 2048), and the words of a hidden vector per thread.
#ifndef LQ8_LMU
#define LQ8_LMU 4
#endif
#ifndef LQ8_LMS
#define LQ8_LMS 3
#endif
constexpr int LMU = LQ8_LMU;   // lm_head: block pairs per streamed unit of a tile (a power of two)
constexpr int LMS = LQ8_LMS;   // lm_head: units in a wave's ring (LMS - 1 in flight while one is summed)
#ifndef LQ8_LMD
#define LQ8_LMD 4
#endif
constexpr int LMD = LQ8_LMD;   // lm_head: chunks per interleaved dot (divides LMU)
constexpr int RSRC_RAW = 0x00020000;  // raw buffer resource, 32-bit data format
constexpr int AUX_NT = 2;      // buffer load cache policy: nontemporal

// The argument block and the layer table, read through the constant address
// space: the kernel never writes them, and so their fields are scalar loads
// (uniform values in SGPRs) even after the kernel's own global stores.
typedef __attribute__((address_space(4))) const PersistArgs CArgs;
typedef __attribute__((address_space(4))) const PLayer CLayer;

// The argument block as a value produced here: its fields are loaded again
// (scalar cache) where they are used instead of being held in registers
// across the whole kernel.
__device__ __forceinline__ CArgs* opaque_args(const PersistArgs* p) {
    CArgs* q = (CArgs*)p;
    asm volatile("" : "+s"(q));
    return q;
}
__device__ __forceinline__ CLayer& layer_of(CArgs& a, int l) { return ((CLayer*)a.layers)[l]; }

__device__ __forceinline__ void tput(uint64_t* p, float v, unsigned tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t traw(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool tok_tag(uint64_t v, unsigned tag) { return (unsigned)(v >> 32) == tag; }

// The workgroup's abort mark: an LDS word behind a generic pointer.  Its
// reads are flat loads, after which the wave waits for vmcnt(0) -- on this
// chip that counts the wave's outstanding stores too, so a check also waits
// for the write-through of the hand-off words the wave has just published.
// Measured with Qwen3-0.6B (tok/s, interleaved runs): this form 1501, the mark
// addressed as LDS (address space 3, lgkmcnt waits only) 1485, that plus an
// explicit vmcnt(0) drain after every publication 1367, this form without the
// check after P1's join 1484 -- so the checks stay as they are.
typedef volatile int* LdsFlag;

// The abort mark as a wave-uniform value (all lanes read the same LDS word;
// readfirstlane tells the compiler so, keeping the branches on it uniform).
__device__ __forceinline__ bool bad_now(LdsFlag bad) { return __builtin_amdgcn_readfirstlane(*bad) != 0; }

// One poll of a bounded wait: false to go on polling; true (with *bad set)
// once the poll limit is reached or another workgroup raised the abort flag.
__device__ __forceinline__ bool poll_stop(unsigned& spins, unsigned* abort_flag, LdsFlag bad) {
    if (*bad) return true;
    ++spins;
    if ((spins & 63) == 0 && sync_load(abort_flag) != 0) {
        *bad = 1;
        return true;
    }
    if (spins > SYNC_SPIN_LIMIT) {
        __hip_atomic_fetch_or(abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *bad = 1;
        return true;
    }
    __builtin_amdgcn_s_sleep(8);
    return false;
}

// *dst(t, u) = the value of the tagged word src(t, u) once it carries `tag`,
// for every unit u < NW of thread t that ok(t, u) admits.  Every
// thread of the workgroup calls it; a lds_sync() and a look at the abort mark
// follow.  One batch of loads per round: the first round loads every word;
// while some have not landed, one lane of the wave polls one of them and the
// next round loads the wave's missing words again.
template <int NW, typename Ok, typename Src, typename Dst>
__device__ __forceinline__ void tfetch(unsigned tag, Ok ok, Src src, Dst dst, unsigned* abort_flag, LdsFlag bad) {
    unsigned pend = 0;
    {
        const int tid = tid_here();
#pragma unroll
        for (int u = 0; u < NW; u++)
            if (ok(tid, u)) pend |= 1u << u;
    }
    unsigned spins = 0;
    for (;;) {
        // indices recomputed here (not held across the wait)
        const int tid = tid_here(), lane = tid & 63;
        uint64_t v[NW];
#pragma unroll
        for (int u = 0; u < NW; u++)
            if ((pend >> u) & 1) v[u] = traw(src(tid, u));
#pragma unroll
        for (int u = 0; u < NW; u++) {
            if (((pend >> u) & 1) && tok_tag(v[u], tag)) {
                *dst(tid, u) = __uint_as_float((unsigned)v[u]);
                pend &= ~(1u << u);
            }
        }
        const uint64_t waiting = __ballot(pend != 0);
        if (waiting == 0) return;
        if (lane == (int)__builtin_ctzll(waiting)) {
            const uint64_t* p = src(tid, (int)__builtin_ctz(pend));
            while (!tok_tag(traw(p), tag))
                if (poll_stop(spins, abort_flag, bad)) break;
        }
        if (bad_now(bad)) return;
    }
}

// The linear case: words src[0, n) into dst[0, n).
template <int NW>
__device__ __forceinline__ void tfetch_lin(int n, unsigned tag, const uint64_t* src, float* dst, unsigned* abort_flag,
                                           LdsFlag bad) {
    tfetch<NW>(tag, [&](int t, int u) { return t + u * PT < n; }, [&](int t, int u) { return src + t + u * PT; },
               [&](int t, int u) { return dst + t + u * PT; }, abort_flag, bad);
}

// A 16-byte chunk of weight codes (global memory, streamed once: nontemporal)
// and a scale, through global-address-space pointers.
typedef __attribute__((address_space(1))) const u32x4 gchunk;
typedef __attribute__((address_space(1))) const uint16_t gscale;
__device__ __forceinline__ u32x4 chunk_load(const int8_t* p) { return __builtin_nontemporal_load((gchunk*)p); }
__device__ __forceinline__ uint16_t scale_load(const uint16_t* p) { return *(gscale*)p; }

// Element j of row `row` of a tiled Q8_0 weight, dequantized (exact).
__device__ __forceinline__ float q8_elem(const int8_t* codes, const uint16_t* scales, int np, int row, int j) {
    const int tile = row / TILE_ROWS, r = row % TILE_ROWS, b = j >> 5, hf = (j >> 4) & 1;
    const float d = f16_bits_to_f32(scales[scale_off(tile, np, b, r)]);
    return d * (float)codes[code_off(tile, np, b, hf, r) + (j & 15)];
}

// The 16 codes of a chunk, unpacked only where they are used: the empty asm
// keeps the compiler from hoisting the byte unpacking of every prefetched
// chunk next to its load (which would hold 16 registers per chunk).
__device__ __forceinline__ float dot16_pinned(u32x4 c, const float* __restrict__ x) {
    asm volatile("" : "+v"(c.x), "+v"(c.y), "+v"(c.z), "+v"(c.w));
    return dot16(c, x);
}

// N chunk dots at once: N of the GEMV's 16-term fmaf chains (each in its
// order, from +0, as dot16), interleaved step by step so that the dependent
// chains overlap (one chain alone waits on each fma's latency).  LEAN: a
// scheduling barrier before each step's input reads, so that the compiler
// does not hoist all 4 N of them (for the register-bound instances).
template <int N, bool LEAN = false>
__device__ __forceinline__ void dot16xN(const u32x4* c, const float* const* x, float* out) {
    uint32_t w[N][4];
#pragma unroll
    for (int k = 0; k < N; k++) {
        u32x4 ck = c[k];
        asm volatile("" : "+v"(ck.x), "+v"(ck.y), "+v"(ck.z), "+v"(ck.w));
        w[k][0] = ck.x;
        w[k][1] = ck.y;
        w[k][2] = ck.z;
        w[k][3] = ck.w;
    }
    float p[N];
#pragma unroll
    for (int k = 0; k < N; k++) p[k] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (LEAN) __builtin_amdgcn_sched_barrier(0);
        float4 xv[N];
#pragma unroll
        for (int k = 0; k < N; k++) xv[k] = *(const float4*)(x[k] + 4 * i);
#pragma unroll
        for (int k = 0; k < N; k++) p[k] = fmaf((float)(int8_t)(w[k][i] & 0xFF), xv[k].x, p[k]);
#pragma unroll
        for (int k = 0; k < N; k++) p[k] = fmaf((float)(int8_t)((w[k][i] >> 8) & 0xFF), xv[k].y, p[k]);
#pragma unroll
        for (int k = 0; k < N; k++) p[k] = fmaf((float)(int8_t)((w[k][i] >> 16) & 0xFF), xv[k].z, p[k]);
#pragma unroll
        for (int k = 0; k < N; k++) p[k] = fmaf((float)(int8_t)(w[k][i] >> 24), xv[k].w, p[k]);
    }
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = p[k];
}

// ---- GEMV work of one workgroup in a phase ------------------------------------
// NTL (1 or 2) 16-row tiles t0, t1 of a tiled weight (np pairs, nb blocks per
// row) over the block pairs [p0, p0 + npv), cut into G <= PW groups of CH
// consecutive pairs (CH a power of two); wave w takes group w of each tile,
// slot j * CH + i holding pair p0 + w * CH + i of tile j.  The group sums
// meet in the pairwise tree over the groups: together the block tree of the
// GEMV order (gemv_tiles), bit for bit.
struct Job {
    const int8_t* codes;
    const uint16_t* scales;
    int np, nb, t0, t1, p0, npv, G;
};

template <int NS>
struct WRegs {
    u32x4 c[NS];
    uint16_t d[NS];
};

// A register set that a workgroup or wave has no item for: zeros, so that
// every load site ends the life of the set's earlier values (a set kept
// only on some paths stays allocated through every phase in between).
template <int NS>
__device__ __forceinline__ void wregs_clear(WRegs<NS>& R) {
#pragma unroll
    for (int i = 0; i < NS; i++) {
        R.c[i] = u32x4{0u, 0u, 0u, 0u};
        R.d[i] = 0;
    }
}

template <int CH>
__device__ __forceinline__ Job make_job(const int8_t* codes, const uint16_t* scales, int np, int nb, int t0, int t1,
                                        int p0, int npv) {
    return Job{codes, scales, np, nb, t0, t1, p0, npv, (npv + CH - 1) / CH};
}

template <int NTL, int CH>
__device__ __forceinline__ void job_load(const Job& J, WRegs<NTL * CH>& R) {
    const int lane = tid_here() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    const int r = lane & 15, bsel = (lane >> 4) >> 1;
    if (wave >= J.G) {
        if constexpr (CH >= 4) wregs_clear(R);
        return;
    }
#pragma unroll
    for (int j = 0; j < NTL; j++) {
        const int tile = j ? J.t1 : J.t0;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int p = J.p0 + min(wave * CH + i, J.npv - 1);
            R.c[j * CH + i] = chunk_load(J.codes + ((size_t)tile * J.np + p) * CHUNK_BYTES + lane * 16);
            R.d[j * CH + i] = scale_load(J.scales + (size_t)tile * 2 * J.np * 16 + bsel * 16 + r + (size_t)p * 32);
        }
    }
}

// The chunks of one tile of the job into slots S0 .. S0 + CH - 1.
template <int CH, int S0, int NSR>
__device__ __forceinline__ void job_load_tile(const Job& J, int tile, WRegs<NSR>& R) {
    const int lane = tid_here() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    const int r = lane & 15, bsel = (lane >> 4) >> 1;
    if (wave >= J.G) return;
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const int p = J.p0 + min(wave * CH + i, J.npv - 1);
        R.c[S0 + i] = chunk_load(J.codes + ((size_t)tile * J.np + p) * CHUNK_BYTES + lane * 16);
        R.d[S0 + i] = scale_load(J.scales + (size_t)tile * 2 * J.np * 16 + bsel * 16 + r + (size_t)p * 32);
    }
}

// Group sums into gs[(j * G + wave) * 16 + row]; xs holds the input of the
// pair range (xs[(2 (p - p0) + b) * 32 + e] = x[(2 p + b) * 32 + e]).
template <int NTL, int CH>
__device__ __forceinline__ void job_dot(const Job& J, const WRegs<NTL * CH>& R, const float* xs, float* gs) {
    constexpr int NS = NTL * CH, NI = NS < 4 ? NS : (CH >= 4 ? 2 : 4);  // chunks, interleaved NI at a time
    const int lane = tid_here() & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid_here() >> 6);
    const int part = lane >> 4, bsel = part >> 1, half = part & 1;
    if (wave >= J.G) return;
    const int cnt = min(CH, J.npv - wave * CH);  // valid pairs of the wave's group
    float v[NS];
#pragma unroll
    for (int s0 = 0; s0 < NS; s0 += NI) {
        const float* xp[NI];
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int i = (s0 + k) % CH, pr = min(wave * CH + i, J.npv - 1);
            xp[k] = xs + (2 * pr + bsel) * 32 + half * 16;
        }
        float h[NI];
        dot16xN<NI, (CH >= 4)>(&R.c[s0], xp, h);
#pragma unroll
        for (int k = 0; k < NI; k++) {
            const int i = (s0 + k) % CH, pr = min(wave * CH + i, J.npv - 1);
            // h0 + h1: the half-0 lane's sum (even 16-lane row) plus the half-1 lane's
            const LanePair hh = lanes16(h[k]);
            const float vb = (hh.lo + hh.hi) * f16_bits_to_f32(R.d[s0 + k]);
            // level s = 1 of the tree: block 2p (lanes 0..31) + block 2p + 1 (lanes 32..63)
            const LanePair vv = lanes32(vb);
            v[s0 + k] = 2 * (J.p0 + pr) + 1 >= J.nb ? vv.lo : vv.lo + vv.hi;
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < NTL; j++) {
        // the tree levels inside a group (as gemv_tiles: s = 1, 2, ..., i + s < cnt)
#pragma unroll
        for (int s = 1; s < CH; s *= 2)
#pragma unroll
            for (int i = 0; i + s < CH; i += 2 * s)
                if (i + s < cnt) v[j * CH + i] = v[j * CH + i] + v[j * CH + i + s];
        if (lane < 16) gs[(j * J.G + wave) * 16 + lane] = v[j * CH];
    }
}

// Row `lane & 15` of the tile: the pairwise tree over the G (<= PW) group
// sums gs[i * 16 + row], in registers (all G values are read at once, then
// v[i] = v[i] + v[i + s] for s = 1, 2, 4, ..., i + s < G: the group tree of
// the GEMV order).
__device__ __forceinline__ float tile_final(const float* gs, int G) {
    const int col = tid_here() & 15;
    float v[PW];
#pragma unroll
    for (int i = 0; i < PW; i++) v[i] = gs[min(i, G - 1) * 16 + col];  // read unconditionally, used below G
#pragma unroll
    for (int s = 1; s < PW; s *= 2)
#pragma unroll
        for (int i = 0; i + s < PW; i += 2 * s)
            if (i + s < G) v[i] = v[i] + v[i + s];
    return v[0];
}

// The pairwise tree over n (<= N) chunk sums v[0 .. n).
template <int N>
__device__ __forceinline__ float chunk_tree_n(float* v, int n) {
#pragma unroll
    for (int s = 1; s < N; s *= 2)
#pragma unroll
        for (int i = 0; i + s < N; i += 2 * s)
            if (i + s < n) v[i] = v[i] + v[i + s];
    return v[0];
}

// RmsNorm (src/rms_norm.rs:143-176) in the order of the GEMV's XS_RMSNORM
// staging: bf16 inputs; SUM64 of squares (wave 0); inv = 1 / sqrt(sum / k +
// eps); out = bf16((v * inv) * bf16(w)).  norm_prefetch loads the weights
// w[tid + j PT] before the phase's hand-off, so that their latency hides
// behind it.
template <int NWV>
__device__ __forceinline__ void norm_prefetch(const float* w, int k, float (&wv)[NWV]) {
    const int tid = tid_here();
#pragma unroll
    for (int j = 0; j < NWV; j++) wv[j] = tid + j * PT < k ? w[tid + j * PT] : 0.0f;
}

// The RmsNorm of the values hv[j] = v[tid + j PT] (j < NWV) that the
// thread holds (the caller joined them), into xs[0, k), and zero over the
// padding [k, 64 np): the bf16 inputs go to LDS once for the reduction,
// whose lanes read their 16 elements at once before the add chain; the
// normalised values come from the registers.
template <int NWV>
__device__ __forceinline__ void stage_rmsnorm_regs(float (&hv)[NWV], float* xs, int k, int np,
                                                   const float (&wv)[NWV], float eps, float* red) {
    const int tid = tid_here();
#pragma unroll
    for (int j = 0; j < NWV; j++) {
        const int i = tid + j * PT;
        if (i < k) {
            hv[j] = bf16_round(hv[j]);
            xs[i] = hv[j];
        }
    }
    lds_sync();
    if (tid < 64) {
        constexpr int NL = NWV * PT / 64;  // elements per lane, at most
        constexpr int NB = NL < 16 ? NL : 16;  // read in batches of NB
        float acc = 0.0f;
#pragma unroll
        for (int j0 = 0; j0 < NL; j0 += NB) {
            float x[NB];
#pragma unroll
            for (int j = 0; j < NB; j++) x[j] = xs[min(tid + 64 * (j0 + j), k - 1)];  // read unconditionally, used below k
#pragma unroll
            for (int j = 0; j < NB; j++)
                if (tid + 64 * (j0 + j) < k) acc = acc + x[j] * x[j];
        }
        acc = wave_sum64(acc);
        if (tid == 0) red[0] = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)k) + eps));
    }
    lds_sync();
    const float inv = red[0];
#pragma unroll
    for (int j = 0; j < NWV; j++) {
        const int i = tid + j * PT;
        if (i < k) xs[i] = bf16_round((hv[j] * inv) * bf16_round(wv[j]));
    }
    for (int i = k + tid; i < np * 64; i += PT) xs[i] = 0.0f;
    lds_sync();
}

// zero the padding block of an odd block count (xs[k, 64 np))
__device__ __forceinline__ void stage_pad(float* xs, int k, int np) {
    for (int i = k + tid_here(); i < np * 64; i += PT) xs[i] = 0.0f;
}

// Greedy pick over the workgroup: (bv, bi) of every thread -> the maximum,
// last index on ties, in every thread.  lds: PW floats + PW ints.
__device__ __forceinline__ void wg_argmax(float& bv, int& bi, float* pv, int* pi) {
    const int tid = tid_here(), lane = tid & 63, wave = tid >> 6;
    argmax_step<32>(bv, bi);
    argmax_step<16>(bv, bi);
    argmax_step<8>(bv, bi);
    argmax_step<4>(bv, bi);
    argmax_step<2>(bv, bi);
    argmax_step<1>(bv, bi);
    if (lane == 0) {
        pv[wave] = bv;
        pi[wave] = bi;
    }
    lds_sync();
    bv = pv[0];
    bi = pi[0];
    for (int q = 1; q < PW; q++)
        if (pv[q] > bv || (pv[q] == bv && pi[q] > bi)) {
            bv = pv[q];
            bi = pi[q];
        }
}

// LDS writes of a wave visible to the wave's own later reads
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The segment combine of kv head g's G query heads (the order of the o GEMV's
// XS_ATTN staging): per head, in segment order, m' = max(m, m_c),
// a_c = exp(m - m'), b_c = exp(m_c - m'), den = den a_c + b_c l_c; per
// element num = num a_c + b_c o_c; x = num / den, published to attl (heads
// concatenated).  Run by the attention item of the newest segment (C - 1),
// which holds that segment's partials itself (own_ml: its (m_c, l_c) per
// head in LDS; own: its o_c elements in registers) and reads the other
// segments' as tagged words.  Segments go in batches of at most CMB_SEGS,
// as many as have their (m_c, l_c) words in NW_ML words per thread: the
// batch's (m_c, l_c) words and the o_c words of its first round arrive in
// one fetch; per head one wave takes the batch's running maximum in order
// (lane 0), the coefficients in parallel (lane j: segment j), then den in
// order (lane 0); each thread carries up to CMB_EK output elements
// (tid + k PT) through the batch, NW_OC o_c words per round.
// LDS (cm): ml [CMB_SEGS][G][2] (m_c, l_c), cf [CMB_SEGS][G][2] (a_c, b_c),
// st [G][2] (running m, den).  false: the launch is aborting.
template <typename Mark>
__device__ __forceinline__ bool combine_heads(unsigned tag, int C, int g, int G, int NH, const uint64_t* partb,
                                              uint64_t* attl, float* cm, const float* own_ml,
                                              const float (&own)[CMB_EK], unsigned* abort_flag,
                                              LdsFlag bad, Mark mark) {
    const int tid = tid_here(), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float* ml = cm;
    float* cf = ml + CMB_SEGS * 2 * G;
    float* st = cf + CMB_SEGS * 2 * G;
    const int GE = G * 128;                            // output elements
    const int EK = (GE + PT - 1) / PT;                 // elements per thread (<= CMB_EK)
    int SBs = 0;                                       // log2 of the segments per o_c round
    while ((2 << SBs) * EK <= NW_OC) SBs++;            // (the largest power of two with EK of them <= NW_OC)
    const int SBm = (1 << SBs) - 1;
    const int cown = C - 1;                            // the combiner's own segment
    const int BS = min(CMB_SEGS, NW_ML * PT / (2 * G));  // segments per batch
    const uint64_t* pb = partb + (size_t)(g * G) * ATT_PART_STRIDE;
    const size_t segw = (size_t)NH * ATT_PART_STRIDE;  // words per segment
    float num[CMB_EK];
#pragma unroll
    for (int k = 0; k < CMB_EK; k++) num[k] = 0.0f;
    if (tid < G) {
        st[2 * tid] = -__builtin_huge_valf();
        st[2 * tid + 1] = 0.0f;
    }
    // o_c unit u of a round starting at segment cb + sb: element tid + (u >> SBs) PT of segment
    // cb + sb + (u & SBm); the own segment's come from registers
    auto oc_ok = [&](int t, int u, int cb, int sb, int nc) {
        const int k = u >> SBs, j = u & SBm;
        return k < EK && t + k * PT < GE && sb + j < nc && cb + sb + j != cown;
    };
    auto oc_src = [&](int t, int u, int cb, int sb) {
        const int k = u >> SBs, j = u & SBm, e = t + k * PT;
        return pb + (size_t)(cb + sb + j) * segw + (e >> 7) * ATT_PART_STRIDE + (e & 127);
    };
    auto oc_update = [&](const float* ov, int cb, int sb, int nc) {
        const int t = tid_here();
#pragma unroll
        for (int u = 0; u < NW_OC; u++) {
            const int k = u >> SBs, j = u & SBm, e = t + k * PT;
            if (k < EK && e < GE && sb + j < nc) {
                float o = ov[u];
#pragma unroll
                for (int kk = 0; kk < CMB_EK; kk++)
                    if (kk == k && cb + sb + j == cown) o = own[kk];
                const int q = ((sb + j) * G + (e >> 7)) * 2;
                const float add = cf[q + 1] * o;
#pragma unroll
                for (int kk = 0; kk < CMB_EK; kk++)
                    if (kk == k) num[kk] = num[kk] * cf[q] + add;
            }
        }
    };
    for (int cb = 0; cb < C; cb += BS) {
        const int nc = min(BS, C - cb);
        // the batch's (m_c, l_c) words (i = (j G + h) 2 + {0: m_c, 1: l_c}) and its first o_c round
        float ov[NW_OC];
        tfetch<NW_ML + NW_OC>(
            tag,
            [&](int t, int u) {
                if (u < NW_ML) {
                    const int i = t + u * PT;
                    return i < nc * G * 2 && cb + i / (2 * G) != cown;
                }
                return oc_ok(t, u - NW_ML, cb, 0, nc);
            },
            [&](int t, int u) {
                if (u < NW_ML) {
                    const int i = t + u * PT, j = i / (2 * G), h = (i >> 1) - j * G;
                    return pb + (size_t)(cb + j) * segw + h * ATT_PART_STRIDE + 128 + (i & 1);
                }
                return oc_src(t, u - NW_ML, cb, 0);
            },
            [&](int t, int u) { return u < NW_ML ? ml + t + u * PT : &ov[u - NW_ML]; }, abort_flag, bad);
        if (tid < 2 * G && cown >= cb && cown < cb + nc) ml[(cown - cb) * 2 * G + tid] = own_ml[tid];
        lds_sync();
        if (bad_now(bad)) return false;
        mark(LQ8_PT_P2_COMB_FETCHED);
        for (int h = wave; h < G; h += PW) {
            if (lane == 0) {
                // m before and after each segment, in order
                float m = st[2 * h];
                for (int j = 0; j < nc; j++) {
                    const float mc = ml[(j * G + h) * 2];
                    const float mn = m > mc ? m : mc;
                    cf[(j * G + h) * 2] = m;
                    cf[(j * G + h) * 2 + 1] = mn;
                    m = mn;
                }
                st[2 * h] = m;
            }
            wave_sync();
            if (lane < nc) {
                const int q = (lane * G + h) * 2;
                const float mp = cf[q], mn = cf[q + 1], mc = ml[q];
                cf[q] = expf_cr(mp - mn);
                cf[q + 1] = expf_cr(mc - mn);
            }
            wave_sync();
            if (lane == 0) {
                float den = st[2 * h + 1];
                for (int j = 0; j < nc; j++) {
                    const int q = (j * G + h) * 2;
                    den = den * cf[q] + cf[q + 1] * ml[q + 1];
                }
                st[2 * h + 1] = den;
            }
        }
        lds_sync();
        mark(LQ8_PT_P2_COMB_COEF);
        oc_update(ov, cb, 0, nc);
        for (int sb = SBm + 1; sb < nc; sb += SBm + 1) {
            tfetch<NW_OC>(tag, [&](int t, int u) { return oc_ok(t, u, cb, sb, nc); },
                          [&](int t, int u) { return oc_src(t, u, cb, sb); }, [&](int t, int u) { return &ov[u]; },
                          abort_flag, bad);
            lds_sync();
            if (bad_now(bad)) return false;
            oc_update(ov, cb, sb, nc);
        }
        lds_sync();  // ml and cf are written again by the next batch
    }
    const int t = tid_here();
#pragma unroll
    for (int k = 0; k < CMB_EK; k++) {
        const int e = t + k * PT;
        if (k < EK && e < GE) tput(attl + (size_t)g * GE + e, __fdiv_rn(num[k], st[2 * (e >> 7) + 1]), tag);
    }
    return true;
}

struct Dims {
    int H, I, NH, NKV, G, QD, KD, QKV, npH, nbH, npQ, nbQ, npI, nbI, T1, TH, TI, T6;
};

__device__ __forceinline__ Dims dims_of(CArgs& a) {
    Dims d;
    d.H = a.H; d.I = a.I; d.NH = a.NH; d.NKV = a.NKV; d.G = a.NH / a.NKV;
    d.QD = a.NH * 128; d.KD = a.NKV * 128; d.QKV = d.QD + 2 * d.KD;
    d.nbH = a.H >> 5; d.npH = (d.nbH + 1) >> 1;
    d.nbQ = d.QD >> 5; d.npQ = (d.nbQ + 1) >> 1;
    d.nbI = a.I >> 5; d.npI = (d.nbI + 1) >> 1;
    d.T1 = (d.QKV + 15) / 16; d.TH = d.H / 16; d.TI = d.I / 16; d.T6 = (a.vocab + 15) / 16;
    return d;
}

// Per-phase locals of layer l, derived again in every phase from the opaque
// argument block (so that nothing of them is held across the phases): the
// dimensions, the layer's weights, the LDS regions and the layer's hand-off
// buffers.
#define LAYER_LOCALS                                                                                       \
    CArgs& a = *opaque_args(pa);                                                               \
    const Dims D = dims_of(a);                                                                             \
    const int tid = tid_here(), lane = tid & 63;                                                           \
    const int pos = a.pos0 + s;                                                                            \
    CLayer& Lw = layer_of(a, l);                                                                        \
    float* xs = sm + a.xs_off;                                                                             \
    float* gs = sm + a.gs_off;                                                                             \
    float* red = sm + a.red_off;                                                                           \
    uint64_t* qkvb = a.qkvb + (size_t)l * D.QKV;                                                           \
    uint64_t* partb = a.partb + (size_t)l * a.cmax * D.NH * ATT_PART_STRIDE;                               \
    uint64_t* attl = a.attb + (size_t)l * D.QD;                                                            \
    uint64_t* resl = a.resb + (size_t)l * (1 + a.nchO) * D.H; /* [h_l | o chunk sums] */                   \
    uint64_t* h2b = a.h2b + (size_t)l * (1 + a.nchD) * D.H; /* [h2 | down chunk sums] */                 \
    uint64_t* actb = a.actb + (size_t)l * D.I;                                                             \
    const int n3 = D.TH * a.nchO;                                                                          \
    (void)tid; (void)lane; (void)pos; (void)Lw; (void)xs; (void)gs; (void)red; (void)qkvb; (void)partb;    \
    (void)attl;                                                                                            \
    (void)resl; (void)h2b; (void)actb; (void)n3

// The jobs of the phases' items (HC: pairs per group of a hidden-long tile and
// of an o item; CH5: pairs per group of a down item).
template <int HC>
__device__ __forceinline__ Job job_qkv(CArgs& a, const Dims& D, CLayer& Lw, int t) {
    return make_job<HC>(Lw.qkv_c, Lw.qkv_s, D.npH, D.nbH, t, t, 0, D.npH);
}
template <int HC>
__device__ __forceinline__ Job job_o(CArgs& a, const Dims& D, CLayer& Lw, int it) {
    const int t = it / a.nchO, c = it - t * a.nchO, pc = a.csO >> 1;
    const int p0 = c * pc;
    return make_job<HC>(Lw.o_c, Lw.o_s, D.npQ, D.nbQ, t, t, p0, min(pc, D.npQ - p0));
}
template <int HC>
__device__ __forceinline__ Job job_gu(CArgs& a, const Dims& D, CLayer& Lw, int t) {
    return make_job<HC>(Lw.gu_c, Lw.gu_s, D.npH, D.nbH, t, D.TI + t, 0, D.npH);
}
template <int CH5>
__device__ __forceinline__ Job job_dn(CArgs& a, const Dims& D, CLayer& Lw, int it) {
    const int t = it / a.nchD, c = it - t * a.nchD, p0 = c * a.csD;
    return make_job<CH5>(Lw.dn_c, Lw.dn_s, D.npI, D.nbI, t, t, p0, min(a.csD, D.npI - p0));
}

// P6 of step s: the final RmsNorm, the lm_head tiles (one wave each) and
// the workgroup's greedy pick, published for the next step.  false: the
// launch is aborting.
template <int HC>
__device__ __forceinline__ bool lm_head_phase(const PersistArgs* __restrict__ pa, int w, int s, unsigned tag, float* sm,
                                              LdsFlag bad, float* pick_v, int* pick_i) {
    constexpr int LMQ = HC * PW / LMU;  // lm_head: units per tile, at most
    constexpr int NWG = nw_res<HC>(), NCJ = nch_max<HC>();  // gather words per thread, chunk sums joined
    const int P = gridDim.x;
    [[maybe_unused]] const int l = 0;  // the P6 marks sit in layer 0's row
    PTRACE(LQ8_PT_P6_START);
    CArgs& a = *opaque_args(pa);
    const Dims D = dims_of(a);
    const int tid = tid_here(), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    float* xs = sm + a.xs_off;
    float* red = sm + a.red_off;
    const int t0 = w * PW + wave, tstride = P * PW;
    const int np = D.npH, nb = D.nbH;
    const int r = lane & 15;
    // a wave streams its tiles in units of LMU block pairs through a
    // ring of LMS register sets: unit u sits in set u % LMS, and the
    // loads of units u + 1 .. u + LMS - 1 are in flight while unit u
    // is summed
    const int nq = (np + LMU - 1) / LMU;  // units per tile, <= LMQ
    u32x4 cr[LMS][LMU];
    uint16_t dr[LMS][LMU];
    // buffer loads: one descriptor per table and a 32-bit lane offset,
    // the tile and chunk offsets uniform (no per-chunk pointers)
    const int tiles_alloc = (D.T6 + 1) & ~1;  // rows stored in multiples of 32
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.emb_c, (short)0, (int)((size_t)tiles_alloc * np * CHUNK_BYTES), RSRC_RAW);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.emb_s, (short)0, (int)((size_t)tiles_alloc * 2 * np * 16 * sizeof(uint16_t)), RSRC_RAW);
    auto load_u = [&](int t, int q, u32x4* c, uint16_t* d) {
        const int ln = tid_here() & 63;
        const int vo = ln * 16, vs = (((ln >> 4) >> 1) * 16 + (ln & 15)) * 2;
#pragma unroll
        for (int i = 0; i < LMU; i++) {
            const int p = min(q * LMU + i, np - 1);
            c[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rc, vo, (t * np + p) * CHUNK_BYTES, AUX_NT));
            d[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, vs, (t * 2 * np + 2 * p) * 32, 0);
        }
    };
    // the unit's pair values, summed by the tree levels inside the unit
    auto dot_u = [&](int q, const u32x4* c, const uint16_t* d) {
        const int ln = tid_here() & 63, bs = (ln >> 4) >> 1, hf = (ln >> 4) & 1;
        float v[LMU];
#pragma unroll
        for (int i0 = 0; i0 < LMU; i0 += LMD) {
            const float* xp[LMD];
#pragma unroll
            for (int k = 0; k < LMD; k++) xp[k] = xs + (2 * min(q * LMU + i0 + k, np - 1) + bs) * 32 + hf * 16;
            float h[LMD];
            dot16xN<LMD, HC == 4>(c + i0, xp, h);
#pragma unroll
            for (int k = 0; k < LMD; k++) {
                const int pc = min(q * LMU + i0 + k, np - 1);
                const LanePair hh = lanes16(h[k]);
                const float vb = (hh.lo + hh.hi) * f16_bits_to_f32(d[i0 + k]);
                const LanePair vv = lanes32(vb);
                v[i0 + k] = 2 * pc + 1 >= nb ? vv.lo : vv.lo + vv.hi;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        const int cnt = np - q * LMU;
#pragma unroll
        for (int s2 = 1; s2 < LMU; s2 *= 2)
#pragma unroll
            for (int i = 0; i + s2 < LMU; i += 2 * s2)
                if (i + s2 < cnt) v[i] = v[i] + v[i + s2];
        return v[0];
    };
    const int ntw = t0 < D.T6 ? (D.T6 - t0 + tstride - 1) / tstride : 0;  // the wave's tiles
    const int U = ntw * nq;                                                  // and units
    auto unit_tile = [&](int u) { return t0 + (u / nq) * tstride; };
    auto unit_q = [&](int u) { return u % nq; };
    if constexpr (HC == 2) {
#pragma unroll
        for (int j = 0; j + 1 < LMS; j++)
            if (j < U) load_u(unit_tile(j), unit_q(j), cr[j], dr[j]);
    }
    float nw[HC];
    norm_prefetch(a.final_norm, D.H, nw);
    // the last layer's output: its h2 + the down projection's chunk sums
    const uint64_t* hp = a.h2b + (size_t)(a.L - 1) * (1 + a.nchD) * D.H;
    float* f = sm;  // [1 + nchD][H]
    tfetch_lin<NWG>((1 + a.nchD) * D.H, tag, hp, f, a.abort_flag, bad);
    lds_sync();
    if (bad_now(bad)) return false;
    float hv[HC];
    const int nchD = a.nchD;
#pragma unroll
    for (int j = 0; j < HC; j++) {
        const int r = tid + j * PT;
        if (r < D.H) {
            float v[NCJ];
#pragma unroll
            for (int q = 0; q < NCJ; q++) v[q] = f[(1 + min(q, nchD - 1)) * D.H + r];
            hv[j] = f[r] + chunk_tree_n<NCJ>(v, nchD);
        }
    }
    stage_rmsnorm_regs(hv, xs, D.H, np, nw, a.eps, red);
    if constexpr (HC == 4) {
#pragma unroll
        for (int j = 0; j + 1 < LMS; j++)
            if (j < U) load_u(unit_tile(j), unit_q(j), cr[j], dr[j]);
    }
    PTRACE(LQ8_PT_P6_NORMED);
    float bv = -__builtin_huge_valf();
    int bi = -1;
    float uv[LMQ];  // the tile's unit values (subtrees of LMU pairs)
    for (int u0 = 0; u0 < U; u0 += LMS) {
#pragma unroll
        for (int j = 0; j < LMS; j++) {
            const int u = u0 + j;
            if (u < U) {
                if (u + LMS - 1 < U)
                    load_u(unit_tile(u + LMS - 1), unit_q(u + LMS - 1), cr[(j + LMS - 1) % LMS],
                           dr[(j + LMS - 1) % LMS]);
                const int q = unit_q(u);
                const float vq = dot_u(q, cr[j], dr[j]);
#pragma unroll
                for (int k = 0; k < LMQ; k++)
                    if (k == q) uv[k] = vq;
                if (q == nq - 1) {
                    // the tree levels above the units (pairs LMU, 2 LMU, ... apart)
#pragma unroll
                    for (int s2 = 1; s2 < LMQ; s2 *= 2)
#pragma unroll
                        for (int i = 0; i + s2 < LMQ; i += 2 * s2)
                            if (i + s2 < nq) uv[i] = uv[i] + uv[i + s2];
                    const int row = unit_tile(u) * 16 + r;
                    const bool valid = lane < 16 && row < a.vocab;
                    float tv = valid ? uv[0] : -__builtin_huge_valf();
                    int ti = valid ? row : -1;
                    argmax_step<8>(tv, ti);
                    argmax_step<4>(tv, ti);
                    argmax_step<2>(tv, ti);
                    argmax_step<1>(tv, ti);
                    if (tv > bv || (tv == bv && ti > bi)) {
                        bv = tv;
                        bi = ti;
                    }
                }
            }
        }
    }
    // lanes 0..15 hold the wave's pick (rows of lanes 16..63 were invalid)
    wg_argmax(bv, bi, pick_v, pick_i);
    if (tid == 0) {
        uint64_t* ab = a.argb + (size_t)(tag & 1) * 2 * P;
        tput(ab + 2 * w, bv, tag);
        tput(ab + 2 * w + 1, __uint_as_float((unsigned)bi), tag);
    }
    // the step's one fenced barrier: the workgroup's key/value cache
    // stores of this step are visible to its waves' loads of the next
    __syncthreads();
    PTRACE(LQ8_PT_P6_DONE);
    return true;
}

// The lm_head phase as a call of its own: its registers are allocated apart
// from the layer phases' (the kernel instance for hidden above 1024 holds
// too many of them across the layers for the phase's load ring).
template <int HC>
__device__ __noinline__ bool lm_head_phase_call(const PersistArgs* __restrict__ pa, int w, int s, unsigned tag,
                                                float* sm, LdsFlag bad, float* pick_v, int* pick_i) {
    // the arguments arrive in vector registers: wave-uniform values again
    const uint64_t pu = (uint64_t)(uintptr_t)pa;
    const uint32_t plo = __builtin_amdgcn_readfirstlane((uint32_t)pu);
    const uint32_t phi = __builtin_amdgcn_readfirstlane((uint32_t)(pu >> 32));
    const PersistArgs* pa_u = (const PersistArgs*)(uintptr_t)(((uint64_t)phi << 32) | plo);
    return lm_head_phase<HC>(pa_u, __builtin_amdgcn_readfirstlane(w), __builtin_amdgcn_readfirstlane(s),
                             __builtin_amdgcn_readfirstlane(tag), sm, bad, pick_v, pick_i);
}

// LONG: the kernel instance for steps with more than cdir segments (the
// combining attention items); the other instance has no combine code at all
// (its presence alone, never run, costs the short-context steps about 3 %
// through register allocation), and the host launches each for its steps.
template <int CH5, bool LONG, int HC>
__global__ __launch_bounds__(PT) void k_decode_persistent(const PersistArgs* __restrict__ pa) {
    constexpr int NWG = nw_res<HC>(), NCJ = nch_max<HC>();  // gather words per thread, chunk sums joined
    extern __shared__ __align__(16) float sm[];
    __shared__ int bad_s;
    __shared__ float pick_v[PW];
    __shared__ int pick_i[PW];
    const LdsFlag bad = &bad_s;
    const int P = gridDim.x, w = blockIdx.x;
    if (threadIdx.x == 0) bad_s = 0;
    lds_sync();

    uint32_t tok = 0;
    for (int s = 0; s < pa->steps; s++) {
        CArgs& a = *opaque_args(pa);
        const Dims D = dims_of(a);
        const unsigned tag = a.tag0 + (unsigned)s;
        // layer 0's q|k|v weights, in flight while the token arrives
        WRegs<HC> R1;
        if (w < D.T1) job_load<1, HC>(job_qkv<HC>(a, D, layer_of(a, 0), w), R1);
        else if constexpr (HC == 4) wregs_clear(R1);
        // ---- the step's input token: the previous step's greedy pick (last
        // index on ties) over the workgroups' picks; the first step's from
        // the previous kernel
        if (s == 0) {
            // the previous kernel's pick (the reference's loop as written:
            // the first generated token, also after an earlier launch)
            tok = a.feed_first ? a.tokens_out[0] : *a.d_tok;
        } else {
            float* f = sm;
            tfetch_lin<NW_ARG>(2 * P, tag - 1, a.argb + (size_t)((tag - 1) & 1) * 2 * P, f, a.abort_flag, bad);
            lds_sync();
            if (bad_now(bad)) goto done;
            const int tid = tid_here();
            float bv = tid < P ? f[2 * tid] : -__builtin_huge_valf();
            int bi = tid < P ? (int)__float_as_uint(f[2 * tid + 1]) : -1;
            wg_argmax(bv, bi, pick_v, pick_i);
            const uint32_t picked = (uint32_t)(bi < 0 ? 0 : bi);
            if (w == 0 && tid == 0) a.tokens_out[a.step0 + s - 1] = picked;
            tok = a.feed_first ? a.tokens_out[0] : picked;
            lds_sync();  // f, pick_v, pick_i are read before they are written again
        }

        for (int l = 0; l < pa->L; l++) {
            // ---- P1: h_l, RmsNorm + q|k|v tiles
            if (w < dims_of(*opaque_args(pa)).T1) {
                LAYER_LOCALS;
                PTRACE(LQ8_PT_P1_START);
                float nw[HC], hv[HC];
                norm_prefetch(Lw.in_norm, D.H, nw);
                if (l > 0) {
                    // h_l = h2 of layer l - 1 + its down projection's chunk sums
                    // joined in the block tree; published for this layer's h2
                    const uint64_t* hp = a.h2b + (size_t)(l - 1) * (1 + a.nchD) * D.H;
                    float* f = sm;  // [1 + nchD][H]
                    tfetch_lin<NWG>((1 + a.nchD) * D.H, tag, hp, f, a.abort_flag, bad);
                    lds_sync();
                    if (bad_now(bad)) goto done;
                    PTRACE(LQ8_PT_P1_GATHERED);
                    const int n1 = min(D.T1, P);
                    // the chunk sums are read unconditionally (an index past
                    // nchD reads the last chunk, which chunk_tree_n ignores), so
                    // all of a thread's LDS reads are in flight together
                    const int nchD = a.nchD;
#pragma unroll
                    for (int j = 0; j < HC; j++) {
                        const int r = tid + j * PT;
                        if (r < D.H) {
                            float v[NCJ];
#pragma unroll
                            for (int q = 0; q < NCJ; q++) v[q] = f[(1 + min(q, nchD - 1)) * D.H + r];
                            hv[j] = f[r] + chunk_tree_n<NCJ>(v, nchD);
                            if (r % n1 == w) tput(resl + r, hv[j], tag);
                        }
                    }
                } else {
                    // the embedding row (src/embedding.rs), published as h_0
                    const int n1 = min(D.T1, P);
#pragma unroll
                    for (int j = 0; j < HC; j++) {
                        const int r = tid + j * PT;
                        if (r < D.H) {
                            hv[j] = q8_elem(a.emb_c, a.emb_s, D.npH, (int)tok, r);
                            if (r % n1 == w) tput(resl + r, hv[j], tag);
                        }
                    }
                }
                if (bad_now(bad)) goto done;
                stage_rmsnorm_regs(hv, xs, D.H, D.npH, nw, a.eps, red);
                PTRACE(LQ8_PT_P1_NORMED);
                for (int t = w; t < D.T1; t += P) {
                    const Job J = job_qkv<HC>(a, D, Lw, t);
                    if (t != w) job_load<1, HC>(J, R1);
                    job_dot<1, HC>(J, R1, xs, gs);
                    lds_sync();
                    PTRACE(LQ8_PT_P1_DOT);
                    if (tid < 64) {
                        const float y = tile_final(gs, J.G);
                        const int row = t * 16 + tid;
                        if (tid < 16 && row < D.QKV) tput(qkvb + row, y, tag);
                    }
                    lds_sync();
                }
            }

            // the o tile's weights, in flight through the attention phase
            WRegs<HC> R3;
            {
                LAYER_LOCALS;
                if (w < n3) job_load<1, HC>(job_o<HC>(a, D, Lw, w), R3);
            }

            // ---- P2: attention per (segment, kv head) item; the item of the
            // newest segment combines its kv head's segments
            PTRACE(LQ8_PT_P2_START);
            {
                LAYER_LOCALS;
                const int L1 = pos + 1, C = (L1 + ATT_SEG - 1) / ATT_SEG, G = D.G;
                const int items2 = C * D.NKV;
                float* qs = sm;                   // [G][128]
                float* kn = qs + G * 128;         // [128]
                float* vn = kn + 128;             // [128]
                float* sc = vn + 128;             // [G][64]
                float* mlc = sc + G * ATT_SEG;    // [G][2]
                float* ks = sm + seg_ks_off(G);   // [64][KPAD], later the V rows [64][128]
                float* qraw = ks;                 // the fetched q (G heads), k, v: [G + 2][128]
                for (int it = w; it < items2; it += P) {
                    const int c = it / D.NKV, g = it - c * D.NKV;
                    const int js = c * ATT_SEG, nj = min(ATT_SEG, L1 - js);
                    const bool last = c == C - 1;
                    const int newrow = last ? pos - js : -1;
                    float* Kc = a.kc + l * (size_t)D.NKV * a.max_pos * 128 + (size_t)g * a.max_pos * 128;
                    float* Vc = a.vc + l * (size_t)D.NKV * a.max_pos * 128 + (size_t)g * a.max_pos * 128;
                    float4 kreg[ATT_SEG * 32 / PT], vreg[ATT_SEG * 32 / PT];
                    seg_load<PT, true>(Kc, Vc, js, nj, kreg, vreg);
                    // q/k norm weights and the position's rotation, ahead of the hand-off
                    const float qn0 = Lw.q_norm[lane], qn1 = Lw.q_norm[lane + 64];
                    const float kn0 = Lw.k_norm[lane], kn1 = Lw.k_norm[lane + 64];
                    const float rc = a.cos_t[(size_t)pos * 64 + (lane & ~1)], rs = a.sin_t[(size_t)pos * 64 + (lane & ~1)];
                    // q of the group's heads; k and v only for the segment holding the position
                    const int nq = (last ? G + 2 : G) * 128;
                    tfetch<NW_QKV>(tag, [&](int tt, int u) { return tt + u * PT < nq; },
                           [&](int tt, int u) {
                               const int i = tt + u * PT, t = i >> 7, e = i & 127;
                               return (const uint64_t*)qkvb +
                                      (t < G ? (g * G + t) * 128 : D.QD + (t == G ? 0 : D.KD) + g * 128) + e;
                           },
                           [&](int tt, int u) { return qraw + tt + u * PT; }, a.abort_flag, bad);
                    lds_sync();
                    if (bad_now(bad)) goto done;
                    PTRACE(LQ8_PT_P2_QKV_IN);
                    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
                    for (int t = wave; t < G + 2; t += PW) {
                        if (t >= G && !last) continue;
                        const float x0 = qraw[t * 128 + lane], x1 = qraw[t * 128 + lane + 64];
                        if (t < G) {
                            head_norm_rope_cs(x0, x1, qn0, qn1, rc, rs, a.eps, qs + t * 128);
                        } else if (t == G) {
                            head_norm_rope_cs(x0, x1, kn0, kn1, rc, rs, a.eps, kn);
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
                    lds_sync();
                    PTRACE(LQ8_PT_P2_ROPED);
                    seg_scores<PT, true, true>(kreg, nj, newrow, kn, qs, G, a.scale, ks, sc, mlc);
                    lds_sync();
                    PTRACE(LQ8_PT_P2_SCORES);
                    seg_stage_v<PT, true>(vreg, nj, newrow, vn, ks);
                    lds_sync();
                    // the segment's partials: published, or kept by the
                    // newest segment's item, which combines the kv head's
                    // segments
                    const bool comb = LONG && C > a.cdir && c == C - 1;
                    float own[CMB_EK];
#pragma unroll
                    for (int k = 0; k < CMB_EK; k++) {
                        const int t = tid + k * PT;
                        own[k] = 0.0f;
                        if (t < G * 128) {
                            const int h = t >> 7, d = t & 127;
                            const float o = pv_chain(sc + h * ATT_SEG, ks, d, nj);
                            own[k] = o;
                            if (!comb) {
                                uint64_t* p = partb + ((size_t)c * D.NH + g * G + h) * ATT_PART_STRIDE;
                                tput(p + d, o, tag);
                                if (d == 0) {
                                    tput(p + 128, mlc[2 * h], tag);
                                    tput(p + 129, mlc[2 * h + 1], tag);
                                }
                            }
                        }
                    }
                    PTRACE(LQ8_PT_P2_PARTIALS);
                    lds_sync();
                    if constexpr (LONG) {
                        if (comb) {
                            // the combine works in the key rows' region (free now); mlc stays
                            if (!combine_heads(tag, C, g, G, D.NH, partb, attl, ks, mlc, own, a.abort_flag, bad,
                                               [&](int pt) { (void)pt; PTRACE(pt); }))
                                goto done;
                            PTRACE(LQ8_PT_P2_COMBINED);
                            lds_sync();
                        }
                    }
                }
            }

            // ---- P3: o tile over one input chunk of the attention output
            // (combined here from the segment partials of the chunk's heads
            // while a step has at most cdir segments, else published by the
            // combining attention items) -> chunk sums
            PTRACE(LQ8_PT_P3_START);
            {
                LAYER_LOCALS;
                const int L1 = pos + 1, C = (L1 + ATT_SEG - 1) / ATT_SEG;
                for (int it = w; it < n3; it += P) {
                    const Job J = job_o<HC>(a, D, Lw, it);
                    if (it != w) job_load<1, HC>(J, R3);
                    const int t = it / a.nchO, c = it - t * a.nchO;
                    const int i0 = J.p0 * 64, rng = min(J.npv * 64, D.QD - i0);
                    if (C <= a.cdir) {
                        const int hA = i0 >> 7, nh = ((i0 + rng - 1) >> 7) - hA + 1;
                        // the partials of the chunk's heads: per segment one run
                        // of R = nh * ATT_PART_STRIDE words (per head o_c[128],
                        // m_c, l_c, 2 unused); word i of the [C][R] staging is
                        // unit (i - tt) / PT of thread tt
                        const int R = nh * ATT_PART_STRIDE;
                        float* pr = sm;                   // [C][R] the runs
                        float* coef = pr + C * R;         // [C][nh][2]: a_c, b_c
                        float* dens = coef + 2 * C * nh;  // [nh]
                        const uint64_t* run0 = partb + (size_t)hA * ATT_PART_STRIDE;
                        const size_t seg_words = (size_t)D.NH * ATT_PART_STRIDE;
                        // i / R as a multiply-high by ceil(2^32 / R): exact for
                        // i < 2^13 and R < 2^19 (the error term stays below 1 / R)
                        const unsigned Rm = 0xFFFFFFFFu / (unsigned)R + 1u;
                        tfetch<NW_PART>(tag,
                                        [&](int tt, int u) {
                                            const int i = tt + u * PT;
                                            const int k = i - (int)__umulhi((unsigned)i, Rm) * R;
                                            return i < C * R && k % ATT_PART_STRIDE < 130;
                                        },
                                        [&](int tt, int u) {
                                            const int i = tt + u * PT, q = (int)__umulhi((unsigned)i, Rm);
                                            return run0 + (size_t)q * seg_words + (i - q * R);
                                        },
                                        [&](int tt, int u) { return pr + tt + u * PT; }, a.abort_flag, bad);
                        lds_sync();
                        if (bad_now(bad)) goto done;
                        PTRACE(LQ8_PT_P3_STAGED);
                        // the combine (combine_heads' order): per head, in
                        // segment order, m' = max(m, m_c), a_c = exp(m - m'),
                        // b_c = exp(m_c - m'), den = den a_c + b_c l_c; per
                        // element num = num a_c + b_c o_c, x = num / den
                        // one wave per head (nh <= PW), lane j holding segment j
                        // (C <= cdir < 64): every lane follows the running
                        // maximum and then den in segment order over the
                        // values read from their lanes, and each computes its
                        // own segment's a_j, b_j
                        {
                            const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
                            if (wave < nh) {
                                const int h = wave;
                                const float mc = lane < C ? pr[lane * R + h * ATT_PART_STRIDE + 128] : 0.0f;
                                const float lc = lane < C ? pr[lane * R + h * ATT_PART_STRIDE + 129] : 0.0f;
                                float m = -__builtin_huge_valf(), mp = 0.0f, mn = 0.0f;
                                for (int cc = 0; cc < C; cc++) {
                                    const float mcc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mc), cc));
                                    const float mx = m > mcc ? m : mcc;
                                    if (lane == cc) {
                                        mp = m;
                                        mn = mx;
                                    }
                                    m = mx;
                                }
                                const float ea = lane < C ? expf_cr(mp - mn) : 0.0f;
                                const float eb = lane < C ? expf_cr(mc - mn) : 0.0f;
                                if (lane < C) {
                                    coef[2 * (lane * nh + h)] = ea;
                                    coef[2 * (lane * nh + h) + 1] = eb;
                                }
                                float den = 0.0f;
                                for (int cc = 0; cc < C; cc++) {
                                    const float a_c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ea), cc));
                                    const float b_c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(eb), cc));
                                    const float l_c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lc), cc));
                                    den = den * a_c + b_c * l_c;
                                }
                                if (lane == 0) dens[h] = den;
                            }
                        }
                        lds_sync();
                        for (int k = tid; k < rng; k += PT) {
                            const int hh = ((i0 + k) >> 7) - hA;
                            float num = 0.0f;
                            for (int cc = 0; cc < C; cc++)
                                num = num * coef[2 * (cc * nh + hh)] +
                                      coef[2 * (cc * nh + hh) + 1] * pr[cc * R + hh * ATT_PART_STRIDE + ((i0 + k) & 127)];
                            xs[k] = __fdiv_rn(num, dens[hh]);
                        }
                        PTRACE(LQ8_PT_P3_COMBINED);
                    } else {
                        tfetch_lin<NW_ATT>(rng, tag, attl + i0, xs, a.abort_flag, bad);
                        lds_sync();
                        if (bad_now(bad)) goto done;
                        PTRACE(LQ8_PT_P3_STAGED);
                    }
                    stage_pad(xs, rng, J.npv);
                    lds_sync();
                    job_dot<1, HC>(J, R3, xs, gs);
                    lds_sync();
                    if (tid < 64) {
                        const float y = tile_final(gs, J.G);
                        if (tid < 16) tput(resl + (size_t)(1 + c) * D.H + t * 16 + tid, y, tag);
                    }
                    lds_sync();
                }
            }

            // the gate|up and down weights, in flight through the hand-offs
            WRegs<2 * HC> R4;
            WRegs<CH5> R5;
            {
                LAYER_LOCALS;
                if (w < D.TI) {
                    const Job J = job_gu<HC>(a, D, Lw, w);
                    if constexpr (HC == 4) job_load_tile<HC, 0>(J, J.t0, R4);  // the up half after the hand-off
                    else job_load<2, HC>(J, R4);
                }
                if (HC == 2 && w < D.TH * a.nchD) job_load<1, CH5>(job_dn<CH5>(a, D, Lw, w), R5);
            }

            // ---- P4: h2 = h_l + o, RmsNorm(h2) + gate / up tile pair -> silu(gate) * up
            {
                LAYER_LOCALS;
            PTRACE(LQ8_PT_P4_START);
            for (int t = w; t < D.TI; t += P) {
                const Job J = job_gu<HC>(a, D, Lw, t);
                if (t != w) job_load<2, HC>(J, R4);
                float* f = sm;  // [1 + nchO][H]
                if (t == w) {
                    float nw[HC];
                    norm_prefetch(Lw.post_norm, D.H, nw);
                    tfetch_lin<NWG>((1 + a.nchO) * D.H, tag, resl, f, a.abort_flag, bad);
                    lds_sync();
                    if (bad_now(bad)) goto done;
                    if constexpr (HC == 4) job_load_tile<HC, HC>(J, J.t1, R4);
                    PTRACE(LQ8_PT_P4_STAGED);
                    const int n4 = min(D.TI, P), nchO = a.nchO;
                    float hv[HC];
#pragma unroll
                    for (int j = 0; j < HC; j++) {
                        const int r = tid + j * PT;
                        if (r < D.H) {
                            float v[NCJ];
#pragma unroll
                            for (int q = 0; q < NCJ; q++) v[q] = f[(1 + min(q, nchO - 1)) * D.H + r];
                            hv[j] = f[r] + chunk_tree_n<NCJ>(v, nchO);
                            if (r % n4 == w) tput(h2b + r, hv[j], tag);
                        }
                    }
                    stage_rmsnorm_regs(hv, xs, D.H, D.npH, nw, a.eps, red);
                    PTRACE(LQ8_PT_P4_NORMED);
                }
                job_dot<2, HC>(J, R4, xs, gs);
                lds_sync();
                PTRACE(LQ8_PT_P4_DOT);
                if (tid < 64) {
                    const float g = tile_final(gs, J.G), u = tile_final(gs + J.G * 16, J.G);
                    if (tid < 16) tput(actb + t * 16 + tid, silu_mul(g, u), tag);
                }
                lds_sync();
            }

            }

            // the next layer's q|k|v weights, in flight through the down projection
            {
                LAYER_LOCALS;
                if (HC == 4 && w < D.TH * a.nchD) job_load<1, CH5>(job_dn<CH5>(a, D, Lw, w), R5);
                if (HC == 2 && l + 1 < a.L && w < D.T1) job_load<1, HC>(job_qkv<HC>(a, D, layer_of(a, l + 1), w), R1);
            }

            // ---- P5: down tile over one input chunk -> chunk sums (the
            // next layer's RMSNorm stage joins them and adds the residual h2)
            {
                LAYER_LOCALS;
            PTRACE(LQ8_PT_P5_START);
            for (int it = w; it < D.TH * a.nchD; it += P) {
                const Job J = job_dn<CH5>(a, D, Lw, it);
                if (it != w) job_load<1, CH5>(J, R5);
                const int t = it / a.nchD, c = it - t * a.nchD;
                // the chunk's input: silu(gate) * up elements [64 p0, 64 (p0 + npv)) within I
                const int i0 = J.p0 * 64, nx = min(J.npv * 64, D.I - i0);
                tfetch_lin<NW_ACT>(nx, tag, (const uint64_t*)actb + i0, xs, a.abort_flag, bad);
                stage_pad(xs, nx, J.npv);
                lds_sync();
                if (bad_now(bad)) goto done;
                PTRACE(LQ8_PT_P5_STAGED);
                job_dot<1, CH5>(J, R5, xs, gs);
                lds_sync();
                if (tid < 64) {
                    const float acc = tile_final(gs, J.G);
                    if (tid < 16) tput(h2b + (size_t)(1 + c) * D.H + t * 16 + tid, acc, tag);
                }
                lds_sync();
                PTRACE(LQ8_PT_P5_DONE);
            }
            }
            if constexpr (HC == 4) {
                // the next layer's q|k|v weights, in flight through its hand-off
                LAYER_LOCALS;
                if (l + 1 < a.L && w < D.T1) job_load<1, HC>(job_qkv<HC>(a, D, layer_of(a, l + 1), w), R1);
                else wregs_clear(R1);
            }
        }

        // ---- P6: final RmsNorm, lm_head tiles (one wave each), greedy pick
        if constexpr (HC == 4) {
            if (!lm_head_phase_call<HC>(pa, w, s, tag, sm, bad, pick_v, pick_i)) goto done;
        } else {
            if (!lm_head_phase<HC>(pa, w, s, tag, sm, bad, pick_v, pick_i)) goto done;
        }
    }

    // the last step's token, and the decode state for the next call
    if (w == 0) {
        CArgs& a = *opaque_args(pa);
        const unsigned tag = a.tag0 + (unsigned)a.steps - 1;
        float* f = sm;
        tfetch_lin<NW_ARG>(2 * P, tag, a.argb + (size_t)(tag & 1) * 2 * P, f, a.abort_flag, bad);
        lds_sync();
        if (bad_now(bad)) goto done;
        const int tid = tid_here();
        float bv = tid < P ? f[2 * tid] : -__builtin_huge_valf();
        int bi = tid < P ? (int)__float_as_uint(f[2 * tid + 1]) : -1;
        wg_argmax(bv, bi, pick_v, pick_i);
        if (tid == 0) {
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

bool persist_layout(const PersistShape& s, int P, PersistLayout* out) {
    if (s.head_dim != 128 || s.NKV <= 0 || s.NH <= 0 || s.NH % s.NKV || s.max_pos <= 0 || P <= 0) return false;
    const int G = s.NH / s.NKV;
    if (G > ATT_MAX_GROUP) return false;
    // hidden <= 2048: a q|k|v, gate/up or lm_head tile (<= 32 block pairs)
    // is one group of hc pairs per wave (the kernel instance's HC: 2 up to
    // hidden 1024, else 4), the lm_head tile fits the units of a wave's
    // ring (hc PW pairs), and a hidden vector is hc words per thread; the
    // attention output (NH * 128) is at most one P3 fetch (NW_ATT words per
    // thread)
    if (s.H % 32 || s.H < 32 || s.H > 2048 || s.I % 32 || s.I < 32 || s.I > 65536 || s.NH * 128 > 2048) return false;
    const int hc = persist_pairs_per_wave(s.H);
    const int QD = s.NH * 128, nbQ = QD / 32, TH = s.H / 16;
    const int npH = (s.H / 32 + 1) / 2, npI = (s.I / 32 + 1) / 2;
    if (npH > hc * PW || s.H > hc * PT || QD > NW_ATT * PT) return false;
    const int cap = (hc == 4 ? NW_RES4 : NW_RES) * PT;  // words of one gather of a hidden vector and its chunk sums
    const int nchm = hc == 4 ? NCH4 : PERSIST_NCH;       // chunk sums one element joins, at most
    // o input chunks: the smallest power-of-two block count whose items fit
    // the workgroups (or one chunk over the whole input, or the widest chunk
    // a workgroup's waves hold: then a workgroup takes several items).  A
    // chunk covers at most PW heads (4 PW blocks): P3's own segment combine
    // runs one wave per head of the chunk.
    int csO = 2;
    auto nch_of = [&](int cs) { return (nbQ + cs - 1) / cs; };
    while (csO < nbQ && csO < std::min(2 * hc * PW, 4 * PW) &&
           (TH * nch_of(csO) > P || nch_of(csO) > nchm || (1 + nch_of(csO)) * s.H > cap))
        csO *= 2;
    const int nchO = nch_of(csO);
    const int pairsO = (std::min(csO, nbQ) + 1) / 2;  // pairs of the widest o chunk
    // P4 gathers h and the o chunk sums; a chunk's pairs are one group per wave
    if (nchO > nchm || (1 + nchO) * s.H > cap || pairsO > hc * PW || std::min(csO, nbQ) > 4 * PW) return false;
    // down input chunks: the smallest power-of-two pair count, at least one
    // pair per wave, whose (tile, chunk) items fit the workgroups (or one
    // chunk over the whole input)
    int csD = PW;
    auto nchd_of = [&](int cs) { return (npI + cs - 1) / cs; };
    while (csD < npI &&
           (TH * nchd_of(csD) > P || nchd_of(csD) > nchm || (1 + nchd_of(csD)) * s.H > cap))
        csD *= 2;
    const int nchD = nchd_of(csD);
    // P1 and P6 gather h2 and the down chunk sums; a down item's pairs are
    // CH5 = csD / PW per wave (a kernel variant for CH5 = 1, 2, 4, 8); its
    // input chunk is one P5 fetch
    if (nchD > nchm || (1 + nchD) * s.H > cap || csD > 8 * PW || std::min(csD, npI) * 64 > NW_ACT * PT)
        return false;
    // the picks (2 words per workgroup) are one fetch; an attention item's
    // q, k, v one more; a combine batch's (m_c, l_c) and a thread's output
    // elements fit their fetches (with a round's o_c words: at most 32)
    if (2 * P > NW_ARG * PT || (G + 2) * 128 > NW_QKV * PT || 2 * G > NW_ML * PT || G * 128 > CMB_EK * PT ||
        NW_ML + NW_OC > 32)
        return false;
    PersistLayout L{};
    L.hc = hc;
    L.csO = csO;
    L.nchO = nchO;
    L.csD = csD;
    L.nchD = nchD;
    // P3's own combine: an o chunk touches nhc heads (whole heads, or one),
    // whose partials are R words per segment; it takes the steps with at
    // most cdir segments, those whose [C][R] runs fit one gather
    const int nhc = std::max(1, std::min(csO, nbQ) * 32 / 128), R = nhc * ATT_PART_STRIDE;
    L.cdir = NW_PART * PT / R;
    if (L.cdir < 1) return false;
    // LDS, in floats.  From 0: the gathers (fr: a hidden vector and its
    // chunk sums, the picks, or P3's [cdir][R] runs with their
    // coefficients), the attention item's region (att_floats, holding the
    // separate combine's comb_floats), never in use at once; then the staged
    // GEMV input xs (a hidden vector, an o chunk or a down chunk), the wave
    // group sums gs (two tiles) and red.
    int fr = std::max(std::max((1 + nchO) * s.H, (1 + nchD) * s.H), 2 * P);
    fr = std::max(fr, L.cdir * R + 2 * L.cdir * nhc + nhc);
    L.fr = (fr + 3) & ~3;
    const int xsz = std::max(std::max(npH, std::min(csD, npI)), pairsO) * 64;
    L.xs_off = L.fr;
    L.gs_off = L.xs_off + xsz;
    L.red_off = L.gs_off + 2 * PW * 16;
    const int total = L.red_off + 16;
    L.att_floats = seg_ks_off(G) + ATT_SEG * KPAD;
    // the fetched q, k, v and later the combine's region sit in the key rows' region
    if ((G + 2) * 128 > ATT_SEG * KPAD) return false;
    L.comb_floats = 4 * CMB_SEGS * G + 2 * G;
    if (L.comb_floats > ATT_SEG * KPAD) return false;
    L.smem_bytes = std::max(total, L.att_floats) * (int)sizeof(float);
    if (L.smem_bytes > 64 * 1024) return false;
    L.words = 0;
    if (out) *out = L;
    return true;
}

bool persist_supported(const PersistShape& s, int num_cus) { return persist_layout(s, num_cus, nullptr); }

template <bool LONG, int HC>
const void* persist_kernel(int ch5) {
    return ch5 == 1   ? (const void*)k_decode_persistent<1, LONG, HC>
           : ch5 == 2 ? (const void*)k_decode_persistent<2, LONG, HC>
           : ch5 == 4 ? (const void*)k_decode_persistent<4, LONG, HC>
                      : (const void*)k_decode_persistent<8, LONG, HC>;
}

int persist_pairs_per_wave(int hidden) { return hidden > 64 * 2 * PW ? 4 : 2; }

lq8_status launch_decode_persistent(hipStream_t st, const PersistArgs* d_args, int smem_bytes, int num_wg, int ch5,
                                    int hc, bool long_ctx) {
    const PersistArgs* args = d_args;
    void* kargs[] = {&args};
    const size_t smem = (size_t)smem_bytes;
    if (hc != 2 && hc != 4) return fail(LQ8_ERR_INVALID_ARG, "persistent decode: no kernel for this hidden size");
    const void* k = hc == 2 ? (long_ctx ? persist_kernel<true, 2>(ch5) : persist_kernel<false, 2>(ch5))
                            : (long_ctx ? persist_kernel<true, 4>(ch5) : persist_kernel<false, 4>(ch5));
    hipError_t e = hipLaunchCooperativeKernel(k, dim3((unsigned)num_wg), dim3(PT), kargs, smem, st);
    if (e == hipErrorCooperativeLaunchTooLarge)
        return fail(LQ8_ERR_DEVICE, "persistent decode: the grid cannot be co-resident");
    if (e != hipSuccess) return hip_fail(e, "persistent decode launch");
    return LQ8_OK;
}

}  // namespace lq8

using namespace lq8;

extern "C" lq8_status lq8_persist_plan(const lq8_qwen3_config* cfg, uint32_t num_workgroups, lq8_persist_info* out) {
    if (!cfg || !out) return fail(LQ8_ERR_INVALID_ARG, "null pointer");
    if (num_workgroups == 0 || num_workgroups > 65536) return fail(LQ8_ERR_INVALID_ARG, "num_workgroups must be 1 .. 65536");
    const PersistShape sh{(int)cfg->hidden_size, (int)cfg->intermediate_size, (int)cfg->num_heads,
                          (int)cfg->num_kv_heads, (int)cfg->head_dim, (int)cfg->max_positions};
    *out = lq8_persist_info{};
    PersistLayout L{};
    // sizes beyond int range are not the kernel's
    if (cfg->hidden_size > 65536 || cfg->intermediate_size > 65536 || cfg->num_heads > 65536 ||
        cfg->num_kv_heads > 65536 || cfg->head_dim > 65536 || cfg->max_positions > (1u << 30) ||
        !persist_layout(sh, (int)num_workgroups, &L))
        return LQ8_OK;
    out->supported = 1;
    out->o_chunk_blocks = (uint32_t)L.csO;
    out->o_chunks = (uint32_t)L.nchO;
    out->down_chunk_pairs = (uint32_t)L.csD;
    out->down_chunks = (uint32_t)L.nchD;
    out->lds_bytes = (uint32_t)L.smem_bytes;
    out->lds_gather_floats = (uint32_t)L.fr;
    out->lds_xs_offset = (uint32_t)L.xs_off;
    out->lds_gs_offset = (uint32_t)L.gs_off;
    out->lds_red_offset = (uint32_t)L.red_off;
    out->lds_attention_floats = (uint32_t)L.att_floats;
    out->lds_combine_floats = (uint32_t)L.comb_floats;
    out->direct_segments = (uint32_t)L.cdir;
    return LQ8_OK;
}

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
