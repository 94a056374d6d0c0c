// gemv.hip -- decode-time Q8_0 GEMV (W8A32) for gfx950.
//
// A workgroup owns TPW consecutive 16-row tiles of W and the whole K range,
// so every output is final when the workgroup ends (no cross-workgroup
// reduction: on this chip a device-scope release/acquire costs more than the
// GEMV body).  The K range of a tile is cut into G groups of CH block pairs
// (CH = 1, 2 or 4); the (tile, group) items are spread over the waves.  A wave
// reads a (tile, pair) chunk with one 16-byte load per lane (16 rows x 2
// blocks = 1 KiB, coalesced).
//
// Issue order inside a workgroup: the loads of the input vector first (into
// registers), then the weight loads of the wave's first item, then the input
// transform (RmsNorm, silu * up, attention combine) into LDS.  Memory
// counters complete in issue order, so the transform waits only for the
// input and runs while the weights are in flight; every load is
// unconditional (indices clamped), so all of a wave's loads are in flight
// together.
//
// Summation order per row (the oracle's GEMV order, bit for bit):
//   h0_b = fmaf chain over codes 0..15 of block b, h1_b over codes 16..31
//   (from +0, lane (row, half) computes one of them); v_b = (h0_b + h1_b) * d_b;
//   pairwise tree over blocks: v[i] += v[i + s] for s = 1, 2, 4, ..., i + s < nb.
// Level s = 1 pairs the two blocks of a chunk (lanes l and l ^ 32), the next
// levels run in-lane over the CH pairs of a group, the rest over the group
// sums; every group starts at a multiple of CH (a power of two), so the split
// follows the tree exactly.
#include "gemv_device.h"
#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

namespace {

constexpr int MAX_CH = 4;
constexpr int MAX_WAVES = 16;
constexpr int SP = 4;  // input float4s per thread held in registers (the rest load-and-use)
constexpr int CU = 4;  // attention segments held in registers (256 positions)
constexpr int ATT_CB = 64;  // attention segments whose combine coefficients are in LDS at once (4096 positions)
constexpr int EA = 2;  // attention outputs per thread held in registers

// Input staging, split into the loads (issued before the weights) and the
// transform into LDS xs[0, k) (ends with a barrier).
template <int XS>
struct Stage {
    float4 xv[SP] = {}, wv[SP] = {};
    float mcs[CU] = {}, lcs[CU] = {};
    float ov[EA][CU] = {};
    float4 ov4[CU] = {};  // k <= 4 * threads: outputs 4 t .. 4 t + 3 (one head) of the first CU segments
    float4 pv[4] = {};    // XS_RMSNORM_JOIN: the chunk sums of the thread's first float4

    // XS_RMSNORM_JOIN: base + the pairwise tree over the n (<= 4) chunk sums
    // p[0 .. n) of 4 consecutive elements (the GEMV block tree's upper levels)
    static __device__ __forceinline__ float4 join4(float4 base, float4 (&p)[4], int n) {
#pragma unroll
        for (int st = 1; st < 4; st *= 2)
#pragma unroll
            for (int i = 0; i + st < 4; i += 2 * st)
                if (i + st < n)
                    p[i] = make_float4(p[i].x + p[i + st].x, p[i].y + p[i + st].y, p[i].z + p[i + st].z,
                                       p[i].w + p[i + st].w);
        return make_float4(base.x + p[0].x, base.y + p[0].y, base.z + p[0].z, base.w + p[0].w);
    }

    // Only waves whose 64 threads reach into the input issue its loads (a
    // wave-uniform condition, so no lane-divergent branch around a load).
    __device__ __forceinline__ void load(const GemvArgs& a, int wave) {
        const int tid = threadIdx.x, nt = blockDim.x, k4 = a.k >> 2;
        const float* __restrict__ x = a.x;
        if (XS == XS_PLAIN || XS == XS_RMSNORM || XS == XS_SILU || XS == XS_RMSNORM_JOIN || XS == XS_SILU_PART) {
#pragma unroll
            for (int e = 0; e < SP; e++) {
                if (wave * 64 + e * nt < k4) {
                    const int i4 = min(tid + e * nt, k4 - 1);
                    xv[e] = *(const float4*)(x + 4 * i4);
                    if (XS == XS_RMSNORM || XS == XS_RMSNORM_JOIN) wv[e] = *(const float4*)(a.norm_w + 4 * i4);
                    if (XS == XS_SILU) wv[e] = *(const float4*)(x + a.k + 4 * i4);
                    if (XS == XS_SILU_PART) wv[e] = *(const float4*)(x + a.xk + 4 * i4);
                    if (XS == XS_RMSNORM_JOIN && e == 0) {
#pragma unroll
                        for (int c = 0; c < 4; c++)
                            if (c < a.nparts) pv[c] = *(const float4*)(a.parts + (size_t)c * a.k + 4 * i4);
                    }
                }
            }
        } else {
            // segment indices clamped to the buffer's capacity, not to the
            // position's segment count: these loads do not wait for the
            // position (entries past it are loaded and never used)
            const int H = a.attn_heads;
            const int cl = a.attn_cmax - 1;
            // thread t < CU * H (or < H): (m_c, l_c) of every segment c < CU of
            // head t % H (threads t < H: head t)
            const int nml = CU * H <= nt ? CU * H : H;
            const int h = min(tid, nml - 1) % H;
            if (wave * 64 < nml) {
#pragma unroll
                for (int c = 0; c < CU; c++) {
                    const float* p = x + ((size_t)min(c, cl) * H + h) * ATT_PART_STRIDE;
                    mcs[c] = p[128];
                    lcs[c] = p[129];
                }
            }
            if (a.k <= 4 * nt) {
                // one float4 per segment and thread (a 16-byte load: each vector
                // memory instruction costs the texture path the same whatever
                // its width)
                if (wave * 64 < k4) {
                    const int i = 4 * min(tid, k4 - 1);
#pragma unroll
                    for (int c = 0; c < CU; c++)
                        ov4[c] = *(const float4*)(x + ((size_t)min(c, cl) * H + (i >> 7)) * ATT_PART_STRIDE + (i & 127));
                }
            } else {
#pragma unroll
                for (int e = 0; e < EA; e++) {
                    if (wave * 64 + e * nt < a.k) {
                        const int i = min(tid + e * nt, a.k - 1);
#pragma unroll
                        for (int c = 0; c < CU; c++)
                            ov[e][c] = x[((size_t)min(c, cl) * H + (i >> 7)) * ATT_PART_STRIDE + (i & 127)];
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void finish(const GemvArgs& a, int wave, float* xs, float* red) {
        const int tid = threadIdx.x, nt = blockDim.x, k = a.k, k4 = k >> 2;
        const float* __restrict__ x = a.x;
        if (XS == XS_PLAIN) {
#pragma unroll
            for (int e = 0; e < SP; e++)
                if (wave * 64 + e * nt < k4 && tid + e * nt < k4) {
                    const float4 v = xv[e];  // component copy: keeps xv in registers
                    *(float4*)(xs + 4 * (tid + e * nt)) = make_float4(v.x, v.y, v.z, v.w);
                }
            for (int i4 = tid + SP * nt; i4 < k4; i4 += nt) *(float4*)(xs + 4 * i4) = *(const float4*)(x + 4 * i4);
            __syncthreads();
        } else if (XS == XS_SILU || XS == XS_SILU_PART) {
            // silu(gate) * up (src/mlp.rs:151-164; silu src/tensor.rs:1978)
            const int uo = XS == XS_SILU ? k : a.xk;  // up's offset from gate
#pragma unroll
            for (int e = 0; e < SP; e++)
                if (wave * 64 + e * nt < k4 && tid + e * nt < k4) {
                    const float4 g = xv[e], u = wv[e];
                    *(float4*)(xs + 4 * (tid + e * nt)) =
                        make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w));
                }
            for (int i4 = tid + SP * nt; i4 < k4; i4 += nt) {
                const float4 g = *(const float4*)(x + 4 * i4), u = *(const float4*)(x + uo + 4 * i4);
                *(float4*)(xs + 4 * i4) =
                    make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w));
            }
            __syncthreads();
        } else if (XS == XS_RMSNORM || XS == XS_RMSNORM_JOIN) {
            // RmsNorm (src/rms_norm.rs:143-176): input rounded to bf16; sum of
            // squares in the SUM64 order (lane l adds elements l, l + 64, ... in
            // order; the 64 partials fold at distances 32, 16, 8, 4, 2, 1);
            // inv = 1 / sqrt(sum / k + eps); out = bf16((v * inv) * bf16(w)).
            // XS_RMSNORM_JOIN: the input is x + the tree over the chunk sums,
            // stored to h_out by workgroup 0 (the residual of the next steps).
            if constexpr (XS == XS_RMSNORM_JOIN) {
                const bool keep = blockIdx.x == 0 && blockIdx.y == 0;
#pragma unroll
                for (int e = 0; e < SP; e++)
                    if (wave * 64 + e * nt < k4 && tid + e * nt < k4) {
                        float4 p[4];
#pragma unroll
                        for (int c = 0; c < 4; c++) {
                            if (e == 0) p[c] = pv[c];
                            else if (c < a.nparts) p[c] = *(const float4*)(a.parts + (size_t)c * k + 4 * (tid + e * nt));
                            else p[c] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                        }
                        const float4 v = join4(xv[e], p, a.nparts);
                        if (keep) *(float4*)(a.h_out + 4 * (tid + e * nt)) = v;
                        *(float4*)(xs + 4 * (tid + e * nt)) = bf16_round4(v);
                    }
                for (int i4 = tid + SP * nt; i4 < k4; i4 += nt) {
                    float4 p[4];
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        p[c] = c < a.nparts ? *(const float4*)(a.parts + (size_t)c * k + 4 * i4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    const float4 v = join4(*(const float4*)(x + 4 * i4), p, a.nparts);
                    if (keep) *(float4*)(a.h_out + 4 * i4) = v;
                    *(float4*)(xs + 4 * i4) = bf16_round4(v);
                }
            } else {
#pragma unroll
                for (int e = 0; e < SP; e++)
                    if (wave * 64 + e * nt < k4 && tid + e * nt < k4) *(float4*)(xs + 4 * (tid + e * nt)) = bf16_round4(xv[e]);
                for (int i4 = tid + SP * nt; i4 < k4; i4 += nt) *(float4*)(xs + 4 * i4) = bf16_round4(*(const float4*)(x + 4 * i4));
            }
            __syncthreads();
            if (tid < 64) {
                float acc = 0.0f;
                for (int i0 = tid; i0 < k; i0 += 64 * 8) {  // 8 LDS reads in flight, then the adds in order
                    float v[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) v[u] = xs[min(i0 + 64 * u, k - 1)];
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        if (i0 + 64 * u < k) acc = acc + v[u] * v[u];
                }
                acc = wave_sum64(acc);
                if (tid == 0) red[0] = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)k) + a.eps));
            }
            __syncthreads();
            const float inv = red[0];
#pragma unroll
            for (int e = 0; e < SP; e++)
                if (wave * 64 + e * nt < k4 && tid + e * nt < k4) {
                    float4* p = (float4*)(xs + 4 * (tid + e * nt));
                    *p = norm4(*p, wv[e], inv);
                }
            for (int i4 = tid + SP * nt; i4 < k4; i4 += nt) {
                float4* p = (float4*)(xs + 4 * i4);
                *p = norm4(*p, *(const float4*)(a.norm_w + 4 * i4), inv);
            }
            __syncthreads();
        } else {
            // Attention output (src/attention.rs:374-399) from per-segment
            // partials (o_c, m_c, l_c) of each head, combined in segment order:
            // m' = max(m, m_c), a = exp(m - m'), b = exp(m_c - m'),
            // num = num * a + b * o_c, den = den * a + b * l_c; x = num / den.
            const int H = a.attn_heads;
            const int C = min(max(a.d_pos ? *a.d_pos : a.pos_base, 0) / ATT_SEG + 1, a.attn_cmax);
            float* coef = red + 4;                     // [min(C, ATT_CB)][H][2]
            float* dens = coef + min(a.attn_cmax, ATT_CB) * H * 2;  // [H]
            if (C <= CU && CU * H <= nt && k <= 4 * nt) {
                // every partial this thread uses is in its registers: the same
                // steps with no global load, so that no wait joins them to the
                // weights issued after the staging's loads.  Thread (segment
                // c, head h) = c * H + h runs its head's running maximum up to
                // c and the two exps of segment c; the combine threads run the
                // denominator chain as they read the coefficients.
                float* lsh = dens + H;  // [CU][H] l_c
                if (tid < CU * H) {
                    const int c = tid / H, h = tid - c * H;
                    float m = -__builtin_huge_valf(), mpc = m, mnc = m, mcc = 0.0f, lcc = 0.0f;
#pragma unroll
                    for (int cc = 0; cc < CU; cc++) {
                        const float mp = m, mv = mcs[cc], lv = lcs[cc];
                        if (cc < C) m = m > mv ? m : mv;
                        const bool me = cc == c;
                        mpc = me ? mp : mpc;
                        mnc = me ? m : mnc;
                        mcc = me ? mv : mcc;
                        lcc = me ? lv : lcc;
                    }
                    if (c < C) {
                        coef[(c * H + h) * 2] = expf_cr(mpc - mnc);
                        coef[(c * H + h) * 2 + 1] = expf_cr(mcc - mnc);
                        lsh[c * H + h] = lcc;
                    }
                }
                __syncthreads();
                if (tid < k4) {
                    const int i = 4 * tid, h = i >> 7;
                    float ca[CU], cb[CU], lc[CU];
#pragma unroll
                    for (int c = 0; c < CU; c++) {
                        const int cc = min(c, C - 1);
                        ca[c] = coef[(cc * H + h) * 2];
                        cb[c] = coef[(cc * H + h) * 2 + 1];
                        lc[c] = lsh[cc * H + h];
                    }
                    float den = 0.0f, n0 = 0.0f, n1 = 0.0f, n2 = 0.0f, n3 = 0.0f;
#pragma unroll
                    for (int c = 0; c < CU; c++)
                        if (c < C) {
                            den = den * ca[c] + cb[c] * lc[c];
                            n0 = n0 * ca[c] + cb[c] * ov4[c].x;
                            n1 = n1 * ca[c] + cb[c] * ov4[c].y;
                            n2 = n2 * ca[c] + cb[c] * ov4[c].z;
                            n3 = n3 * ca[c] + cb[c] * ov4[c].w;
                        }
                    *(float4*)(xs + i) = make_float4(__fdiv_rn(n0, den), __fdiv_rn(n1, den), __fdiv_rn(n2, den),
                                                     __fdiv_rn(n3, den));
                }
                __syncthreads();
            } else {
            // batches of ATT_CB segments (the coefficients of one batch in LDS):
            // each head's running maximum and denominator, and each element's
            // running numerator (in xs), carry from batch to batch, so the
            // chain is the one above whatever the number of segments
            float* mrun = dens + H;  // [H]
            for (int b0 = 0; b0 < C; b0 += ATT_CB) {
                const int b1 = min(b0 + ATT_CB, C);
                for (int h = tid; h < H; h += nt) {
                    float m = b0 == 0 ? -__builtin_huge_valf() : mrun[h], den = b0 == 0 ? 0.0f : dens[h];
                    for (int c0 = b0; c0 < b1; c0 += CU) {
                        float mc[CU], lc[CU];
#pragma unroll
                        for (int c = 0; c < CU; c++) {
                            if (c0 == 0 && h == tid) {
                                mc[c] = mcs[c];
                                lc[c] = lcs[c];
                            } else {
                                const float* p = x + ((size_t)min(c0 + c, C - 1) * H + h) * ATT_PART_STRIDE;
                                mc[c] = p[128];
                                lc[c] = p[129];
                            }
                        }
                        // the running maxima first, then the exps of every segment
                        // (independent of each other), then the denominator chain
                        float mp[CU], mn[CU], ea[CU], eb[CU];
#pragma unroll
                        for (int c = 0; c < CU; c++) {
                            mp[c] = m;
                            if (c0 + c < b1) m = m > mc[c] ? m : mc[c];
                            mn[c] = m;
                        }
#pragma unroll
                        for (int c = 0; c < CU; c++) {
                            ea[c] = expf_cr(mp[c] - mn[c]);
                            eb[c] = expf_cr(mc[c] - mn[c]);
                        }
#pragma unroll
                        for (int c = 0; c < CU; c++) {
                            if (c0 + c < b1) {
                                coef[((c0 - b0 + c) * H + h) * 2] = ea[c];
                                coef[((c0 - b0 + c) * H + h) * 2 + 1] = eb[c];
                                den = den * ea[c] + eb[c] * lc[c];
                            }
                        }
                    }
                    mrun[h] = m;
                    dens[h] = den;
                }
                __syncthreads();
                const bool last = b1 == C;
                for (int e0 = 0; tid + e0 * nt < k; e0 += EA) {
#pragma unroll
                    for (int e = 0; e < EA; e++) {
                        const int i = tid + (e0 + e) * nt;
                        if (i < k) {
                            const int h = i >> 7, d = i & 127;
                            float num = b0 == 0 ? 0.0f : xs[i];
                            for (int c0 = b0; c0 < b1; c0 += CU) {
                                float o[CU], ca[CU], cb[CU];
#pragma unroll
                                for (int c = 0; c < CU; c++) {
                                    const int cc = min(c0 + c, b1 - 1);
                                    o[c] = (c0 == 0 && e0 == 0 && k > 4 * nt)
                                               ? ov[e][c]
                                               : x[((size_t)cc * H + h) * ATT_PART_STRIDE + d];
                                    ca[c] = coef[((cc - b0) * H + h) * 2];  // coefficients read before the chain
                                    cb[c] = coef[((cc - b0) * H + h) * 2 + 1];
                                }
#pragma unroll
                                for (int c = 0; c < CU; c++)
                                    if (c0 + c < b1) num = num * ca[c] + cb[c] * o[c];
                            }
                            xs[i] = last ? __fdiv_rn(num, dens[h]) : num;
                        }
                    }
                }
                __syncthreads();
            }
            }
        }
    }
};

// Pairs per group for a K range of np pairs over up to W waves.
inline int pick_ch(int np, int w) {
    int ch = 1;
    while (ch < MAX_CH && (np + ch - 1) / ch > w) ch *= 2;
    return ch;
}

// TPW tiles from tile0 (ntiles of them valid): rows tile*16 .. tile*16+15.
// LDS: xs [np * 64] (the input, zero over the padding block of an odd nb),
// gs [ntiles * G][16] group sums, red [4] (+ the XS_ATTN coefficients).
template <int XS, int EPI, int CH>
__device__ __forceinline__ void gemv_tiles(const GemvArgs& a, int tile0, int ntiles, float* sm) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar control flow
    const int W = blockDim.x >> 6;
    const int nb = a.k >> 5, np = (nb + 1) >> 1;
    // EPI_PART: the input is one chunk of the weight's rows, from pair pw0
    // of npw (the chunk's sums are subtrees of the GEMV block tree)
    const int npw = EPI == EPI_PART ? a.npw : np;
    const int pw0 = EPI == EPI_PART ? a.p0 : 0;
    const int G = (np + CH - 1) / CH;
    const int items = ntiles * G;
    float* xs = sm;
    float* gs = sm + np * 64;
    float* red = gs + items * 16;
    const int r = lane & 15, part = lane >> 4, bsel = part >> 1, half = part & 1;
    const int8_t* cbase = a.codes + ((size_t)tile0 * npw + pw0) * CHUNK_BYTES + lane * 16;
    const uint16_t* sbase = a.scales + (size_t)tile0 * 2 * npw * 16 + (size_t)pw0 * 32 + bsel * 16 + r;
    Stage<XS> st;
    st.load(a, wave);
    if ((nb & 1) && threadIdx.x < 32) xs[a.k + threadIdx.x] = 0.0f;  // ordered by the staging barriers
    // weights of the current item (cv, ds) and the next one (nv, ns)
    u32x4 cv[CH], nv[CH];
    uint16_t ds[CH], ns[CH];
    {
        const int it0 = min(wave, items - 1);
        const int t0 = it0 / G, g0 = it0 - t0 * G;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int c = t0 * npw + min(g0 * CH + i, np - 1);  // chunk of (tile t0, group g0)
            nv[i] = __builtin_nontemporal_load((const u32x4*)(cbase + (size_t)c * CHUNK_BYTES));
            ns[i] = sbase[(size_t)c * 32];
        }
    }
    st.finish(a, wave, xs, red);
    for (int item = wave; item < items; item += W) {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            cv[i] = nv[i];
            ds[i] = ns[i];
        }
        if (item + W < items) {
            const int tn = (item + W) / G, gn = item + W - tn * G;
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const int c = tn * npw + min(gn * CH + i, np - 1);
                nv[i] = __builtin_nontemporal_load((const u32x4*)(cbase + (size_t)c * CHUNK_BYTES));
                ns[i] = sbase[(size_t)c * 32];
            }
        }
        const int g = item % G;
        const int cnt = min(CH, np - g * CH);  // valid pairs of this group
        float v[CH];
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int p = min(g * CH + i, np - 1);
            const float h = dot16(cv[i], xs + (2 * p + bsel) * 32 + half * 16);
            // h0 + h1: the half-0 lane's sum (even 16-lane row) plus the half-1 lane's
            const LanePair hh = lanes16(h);
            const float vb = (hh.lo + hh.hi) * f16_bits_to_f32(ds[i]);
            // level s = 1 of the tree: v_2p (lanes 0..31) + v_2p+1 (lanes 32..63),
            // v_2p alone when block 2p + 1 is the padding of an odd nb
            const LanePair vv = lanes32(vb);
            v[i] = 2 * p + 1 >= nb ? vv.lo : vv.lo + vv.hi;
        }
#pragma unroll
        for (int s = 1; s < CH; s *= 2)
#pragma unroll
            for (int i = 0; i + s < CH; i += 2 * s)
                if (i + s < cnt) v[i] = v[i] + v[i + s];
        if (lane < 16) gs[item * 16 + lane] = v[0];
    }
    __syncthreads();
    if (wave < ntiles) {
        // wave t finishes tile tile0 + t: the tree over its G group sums
        const float* tg = gs + wave * G * 16;
        float acc = 0.0f;
        if (G <= 16) {
            float t[16];
#pragma unroll
            for (int i = 0; i < 16; i++) t[i] = i < G ? tg[i * 16 + r] : 0.0f;
#pragma unroll
            for (int s = 1; s < 16; s *= 2)
#pragma unroll
                for (int i = 0; i + s < 16; i += 2 * s)
                    if (i + s < G) t[i] = t[i] + t[i + s];
            acc = t[0];
        } else if (lane < 16) {
            float* tw = gs + wave * G * 16;
            for (int s = 1; s < G; s *= 2)
                for (int i = 0; i + s < G; i += 2 * s) tw[i * 16 + lane] = tw[i * 16 + lane] + tw[(i + s) * 16 + lane];
            acc = tw[lane];
        }
        const int tile = tile0 + wave;
        const int row = tile * TILE_ROWS + r;
        const bool valid = lane < 16 && row < a.n;
        if (EPI == EPI_RESID) {
            if (valid) a.y[row] = a.resid[row] + acc;
        } else {
            if (valid) a.y[row] = acc;
        }
        if (EPI == EPI_ARGMAX) {
            // greedy pick within the tile: maximum, last index on ties
            float bv = valid ? acc : -__builtin_huge_valf();
            int bi = valid ? row : -1;
            argmax_step<8>(bv, bi);
            argmax_step<4>(bv, bi);
            argmax_step<2>(bv, bi);
            argmax_step<1>(bv, bi);
            if (lane == 0) {
                a.arg_val[tile] = bv;
                a.arg_idx[tile] = bi;
            }
        }
    }
}

template <int XS, int EPI, int CH>
__global__ __launch_bounds__(1024) void k_gemv(GemvArgs a, int tpw) {
    extern __shared__ float smem[];
    const int tiles = (a.n + TILE_ROWS - 1) / TILE_ROWS;
    const int tile0 = blockIdx.x * tpw;
    if constexpr (EPI == EPI_PART) {
        // chunk blockIdx.y: pairs p0 .. p0 + part_pairs - 1 of the input
        const int npf = ((a.k >> 5) + 1) >> 1, c = blockIdx.y, p0 = c * a.part_pairs;
        const int npv = min(a.part_pairs, npf - p0), e0 = 64 * p0;
        GemvArgs ac = a;
        ac.x = a.x + e0;
        ac.k = min(64 * npv, a.k - e0);
        ac.npw = npf;
        ac.p0 = p0;
        ac.xk = a.k;
        ac.y = a.y + (size_t)c * a.n;
        gemv_tiles<XS, EPI, CH>(ac, tile0, min(tpw, tiles - tile0), smem);
    } else {
        gemv_tiles<XS, EPI, CH>(a, tile0, min(tpw, tiles - tile0), smem);
    }
}

__global__ __launch_bounds__(256) void k_gemv_grouped(const GemvProblemDev* __restrict__ probs, int count) {
    extern __shared__ float smem[];
    int lo = 0, hi = count - 1;
    const int t = blockIdx.x;
    while (lo < hi) {  // the problem owning this tile (tile_begin ascending)
        const int mid = (lo + hi + 1) >> 1;
        if (probs[mid].tile_begin <= t) lo = mid;
        else hi = mid - 1;
    }
    const GemvProblemDev p = probs[lo];
    GemvArgs a{p.codes, p.scales, p.x, nullptr, p.y, nullptr, nullptr, nullptr, p.n, p.k, 0.0f};
    // (descriptor k is bounded by GEMV_MAX_K on the host)
    gemv_tiles<XS_PLAIN, EPI_STORE, MAX_CH>(a, t - p.tile_begin, 1, smem);
}

// ---- inputs longer than the staging limit --------------------------------------
//
// k > GEMV_MAX_K (plain input, plain store): one 16-row tile per workgroup; the input is
// staged LONG_PAIRS block pairs at a time.  LONG_PAIRS is a multiple of
// LONG_CH, so every group of LONG_CH pairs lies inside one stage, and the
// group sums meet in the same pairwise tree as in gemv_tiles: the order (and
// so every bit of y) is the GEMV order of the oracle.
constexpr int LONG_PAIRS = 128;  // 256 blocks = 8192 values = 32 KiB of LDS per stage
constexpr int LONG_CH = 4;
constexpr int LONG_THREADS = 512;

__global__ __launch_bounds__(LONG_THREADS) void k_gemv_long(GemvArgs a) {
    extern __shared__ float smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int W = blockDim.x >> 6;
    const int nb = a.k >> 5, np = (nb + 1) >> 1;
    const int G = (np + LONG_CH - 1) / LONG_CH;
    float* xs = smem;                    // [LONG_PAIRS * 64] the staged stage
    float* gs = xs + LONG_PAIRS * 64;    // [G][16] group sums
    const int tile = blockIdx.x;
    const int r = lane & 15, part = lane >> 4, bsel = part >> 1, half = part & 1;
    const int8_t* cbase = a.codes + (size_t)tile * np * CHUNK_BYTES + lane * 16;
    const uint16_t* sbase = a.scales + (size_t)tile * 2 * np * 16 + bsel * 16 + r;
    for (int p0 = 0; p0 < np; p0 += LONG_PAIRS) {
        const int pairs = min(LONG_PAIRS, np - p0);
        const int e0 = p0 * 64, e1 = min(a.k, (p0 + pairs) * 64);
        // values past k (the padding block of an odd nb) stage as 0
        for (int i4 = threadIdx.x; 4 * i4 < pairs * 64; i4 += blockDim.x) {
            const int e = e0 + 4 * i4;
            *(float4*)(xs + 4 * i4) = e < e1 ? *(const float4*)(a.x + e) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        __syncthreads();
        const int gn = (pairs + LONG_CH - 1) / LONG_CH;
        for (int g = wave; g < gn; g += W) {
            u32x4 cv[LONG_CH];
            uint16_t ds[LONG_CH];
#pragma unroll
            for (int i = 0; i < LONG_CH; i++) {
                const int c = min(p0 + g * LONG_CH + i, np - 1);
                cv[i] = __builtin_nontemporal_load((const u32x4*)(cbase + (size_t)c * CHUNK_BYTES));
                ds[i] = sbase[(size_t)c * 32];
            }
            const int cnt = min(LONG_CH, pairs - g * LONG_CH);
            float v[LONG_CH];
#pragma unroll
            for (int i = 0; i < LONG_CH; i++) {
                const int pl = min(g * LONG_CH + i, pairs - 1);  // pair within the stage
                const float h = dot16(cv[i], xs + (2 * pl + bsel) * 32 + half * 16);
                const LanePair hh = lanes16(h);
                const float vb = (hh.lo + hh.hi) * f16_bits_to_f32(ds[i]);
                const LanePair vv = lanes32(vb);
                v[i] = 2 * (p0 + pl) + 1 >= nb ? vv.lo : vv.lo + vv.hi;
            }
#pragma unroll
            for (int s = 1; s < LONG_CH; s *= 2)
#pragma unroll
                for (int i = 0; i + s < LONG_CH; i += 2 * s)
                    if (i + s < cnt) v[i] = v[i] + v[i + s];
            if (lane < 16) gs[(p0 / LONG_CH + g) * 16 + lane] = v[0];
        }
        __syncthreads();  // the stage is overwritten next; the group sums are read below
    }
    if (wave == 0 && lane < 16) {
        for (int s = 1; s < G; s *= 2)
            for (int i = 0; i + s < G; i += 2 * s) gs[i * 16 + lane] = gs[i * 16 + lane] + gs[(i + s) * 16 + lane];
        const int row = tile * TILE_ROWS + lane;
        if (row < a.n) a.y[row] = gs[lane];
    }
}

// ---- multi-vector GEMV ------------------------------------------------------
//
// One workgroup (4 waves) per (problem, 16-row tile, vector split); with
// EPI_SWIGLU per (problem, tile pair 2i, 2i + 1) of a weight whose tiles
// interleave gate and up by 8 rows (tile t: gate rows 8t .. 8t+7, then up
// rows 8t .. 8t+7), which gives silu(gate) * up of rows 16i .. 16i+15.
// Up to VB input vectors are staged in LDS at a time; a wave takes (tile,
// group of CH pairs) items, unpacks each 16-byte code chunk to floats once
// and runs the GEMV order of gemv_tiles for every staged vector; the group
// sums go to LDS and one thread per (vector, row) runs the tree over the
// groups.  PF: the wave's first item's weights are issued before the input
// staging and every item prefetches the wave's next one (across staging
// passes too).
template <int XS, int EPI, int CH, int VB, bool PF, int NTS>
__global__ __launch_bounds__(256) void k_gemv_mv(MvArgs a) {
    extern __shared__ float smem[];
    // tiles per workgroup: NT consecutive tiles from `tile` (the host keeps
    // tiles % NT == 0; EPI_SWIGLU: the pair 2i, 2i + 1)
    constexpr int NT = EPI == EPI_SWIGLU ? 2 : NTS;
    const int tiles_all = (a.rows + TILE_ROWS - 1) / TILE_ROWS;
    const int tiles_p = tiles_all / NT;
    const int j = blockIdx.x / tiles_p, tile = (blockIdx.x - j * tiles_p) * NT;
    if (j >= (a.n_prob ? *a.n_prob : 1)) return;
    const int e = a.prob_id ? a.prob_id[j] : j;
    const int vbeg = a.vec_begin ? a.vec_begin[j] : 0;
    const int vcnt = a.vec_count ? a.vec_count[j] : a.nvec;
    if ((int)blockIdx.y * VB >= vcnt) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int k = a.k, k4 = k >> 2, nb = k >> 5, np = (nb + 1) >> 1;
    const int G = (np + CH - 1) / CH;
    // a staged vector spans G * CH pairs: a group's chunks past np read this
    // padding (in bounds, values unused) at fixed offsets from the group's first
    const int xstride = G * CH * 64;
    float* xs = smem;                    // [VB][xstride]
    float* gs = xs + VB * xstride;       // [VB][NT][G][16]
    float* red = gs + VB * NT * G * 16;  // [VB]
    const int r = lane & 15, part = lane >> 4, bsel = part >> 1, half = part & 1;
    const size_t gt = (size_t)e * a.prob_tiles + tile;
    const int8_t* cbase = a.codes + gt * np * CHUNK_BYTES + lane * 16;
    const uint16_t* sbase = a.scales + gt * 2 * np * 16 + bsel * 16 + r;
    const size_t cstep = (size_t)np * CHUNK_BYTES, sstep = (size_t)2 * np * 16;  // the next tile
    const int items = NT * G;
    // weights of item `it` (clamped: every load in bounds and unconditional)
    u32x4 pv[CH];
    uint16_t ps[CH];
#define MV_LOAD_ITEM(it_)                                                                                   \
    {                                                                                                       \
        const int itc = min((it_), items - 1), ttc = itc / G, gc = itc - ttc * G;                           \
        _Pragma("unroll") for (int i = 0; i < CH; i++) {                                                    \
            const int c = min(gc * CH + i, np - 1);                                                         \
            pv[i] = __builtin_nontemporal_load((const u32x4*)(cbase + ttc * cstep + (size_t)c * CHUNK_BYTES)); \
            ps[i] = sbase[ttc * sstep + (size_t)c * 32];                                                    \
        }                                                                                                   \
    }
    // norm weights first (4 float4 per thread cover k <= 4096), then the PF
    // weights: memory counters complete in issue order, so the norm weights'
    // early use (their bf16 rounding) does not wait for the codes
    float4 nw[4];
    if (XS == XS_RMSNORM) {
#pragma unroll
        for (int j = 0; j < 4; j++) nw[j] = *(const float4*)(a.norm_w + 4 * min(tid + 256 * j, k4 - 1));
    }
    if (PF) {
        if (XS == XS_RMSNORM) __builtin_amdgcn_sched_barrier(0);
        MV_LOAD_ITEM(wave);
        __builtin_amdgcn_sched_barrier(0);  // the codes ahead of the input staging's waits
    }
    for (int v0 = blockIdx.y * VB; v0 < vcnt; v0 += gridDim.y * VB) {
        const int nv = min(VB, vcnt - v0);
        // ---- stage nv vectors (transform per XS) ----
        for (int v = 0; v < nv; v++) {
            const int ent = vbeg + v0 + v;
            const int slot = a.slots ? a.slots[ent] : ent;
            const float* x = a.x + (size_t)(slot / a.x_div) * a.x_stride;
            float* xv = xs + v * xstride;
            for (int i4 = tid; i4 < k4; i4 += 256) {
                const float4 g = *(const float4*)(x + 4 * i4);
                float4 o;
                if (XS == XS_SILU) {
                    const float4 u = *(const float4*)(x + k + 4 * i4);
                    o = make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w));
                } else if (XS == XS_RMSNORM) {
                    o = bf16_round4(g);
                } else {
                    o = g;
                }
                *(float4*)(xv + 4 * i4) = o;
            }
            if ((nb & 1) && tid < 32) xv[k + tid] = 0.0f;
        }
        __syncthreads();
        if (XS == XS_RMSNORM) {
            // SUM64 order per vector (wave v), as the single-vector staging
            if (wave < nv) {
                const float* xv = xs + wave * xstride;
                float acc = 0.0f;
                for (int i0 = lane; i0 < k; i0 += 64 * 8) {
                    float v[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) v[u] = xv[min(i0 + 64 * u, k - 1)];
#pragma unroll
                    for (int u = 0; u < 8; u++)
                        if (i0 + 64 * u < k) acc = acc + v[u] * v[u];
                }
                acc = wave_sum64(acc);
                if (lane == 0) red[wave] = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)k) + a.eps));
            }
            __syncthreads();
            for (int v = 0; v < nv; v++) {
                const float inv = red[v];
                float* xv = xs + v * xstride;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (tid + 256 * j < k4) {
                        float4* p = (float4*)(xv + 4 * (tid + 256 * j));
                        *p = norm4(*p, nw[j], inv);
                    }
                for (int i4 = tid + 1024; i4 < k4; i4 += 256) {
                    float4* p = (float4*)(xv + 4 * i4);
                    *p = norm4(*p, *(const float4*)(a.norm_w + 4 * i4), inv);
                }
            }
            __syncthreads();
        }
        // ---- items: (tile, group of CH pairs) ----
        for (int it = wave; it < items; it += 4) {
            const int tt = it / G, g = it - tt * G;
            u32x4 cv[CH];
            uint16_t ds[CH];
            if (!PF) MV_LOAD_ITEM(it);
#pragma unroll
            for (int i = 0; i < CH; i++) {
                cv[i] = pv[i];
                ds[i] = ps[i];
            }
            if (PF) {
                // the wave's next item while this one computes: the next of this
                // pass, else the wave's first of the next pass (after the last
                // item a clamped reload: unconditional, so that no wait for it is
                // placed where the paths join)
                const int nx = it + 4 < items || v0 + (int)gridDim.y * VB >= vcnt ? it + 4 : wave;
                MV_LOAD_ITEM(nx);
            }
            const int cnt = min(CH, np - g * CH);
            float dsf[CH];
#pragma unroll
            for (int i = 0; i < CH; i++) dsf[i] = f16_bits_to_f32(ds[i]);
            if constexpr (VB > 1) {
                // Vector pairs (a, b) = (2pp, 2pp + 1) share every lane exchange; a
                // vector left over pairs with itself (b = a, no second chain).
                // Chunk-outer: one chunk's codes are unpacked at a time and used by
                // every staged vector.  After rows16 and the scale, s[pp][i] holds
                // in its rows (a, 2p) (b, 2p) (a, 2p+1) (b, 2p+1) of pair
                // p = g*CH + i; halves32 of s[pp][i] and s[pp][i + CH/2] gives the
                // pair values of chunk i (rows 0, 1) and chunk i + CH/2 (rows 2, 3),
                // so the tree over t[] runs the lower and upper half of the group
                // side by side and the last halves32 adds the halves.  A chunk past
                // np enters as -0.0, which leaves any sum unchanged (a + -0.0 == a
                // bit for bit), so partial groups keep the one-vector order.
                constexpr int NPP = VB / 2;
                float s[NPP][CH];
#pragma unroll
                for (int i = 0; i < CH; i++) {
                    float w[16];
                    const uint32_t w4[4] = {cv[i].x, cv[i].y, cv[i].z, cv[i].w};
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        w[4 * q] = (float)(int8_t)(w4[q] & 0xFF);
                        w[4 * q + 1] = (float)(int8_t)((w4[q] >> 8) & 0xFF);
                        w[4 * q + 2] = (float)(int8_t)((w4[q] >> 16) & 0xFF);
                        w[4 * q + 3] = (float)(int8_t)(w4[q] >> 24);
                    }
                    const int off = (2 * (g * CH + i) + bsel) * 32 + half * 16;
#pragma unroll
                    for (int pp = 0; pp < NPP; pp++) {
                        if (2 * pp >= nv) continue;
                        const float* xa = xs + 2 * pp * xstride + off;
                        float ha = 0.0f, hb = 0.0f;
                        if (2 * pp + 1 < nv) {
                            const float* xb = xa + xstride;
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                const float4 xq = *(const float4*)(xa + 4 * q);
                                const float4 xr = *(const float4*)(xb + 4 * q);
                                ha = fmaf(w[4 * q], xq.x, ha);
                                hb = fmaf(w[4 * q], xr.x, hb);
                                ha = fmaf(w[4 * q + 1], xq.y, ha);
                                hb = fmaf(w[4 * q + 1], xr.y, hb);
                                ha = fmaf(w[4 * q + 2], xq.z, ha);
                                hb = fmaf(w[4 * q + 2], xr.z, hb);
                                ha = fmaf(w[4 * q + 3], xq.w, ha);
                                hb = fmaf(w[4 * q + 3], xr.w, hb);
                            }
                        } else {
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                const float4 xq = *(const float4*)(xa + 4 * q);
                                ha = fmaf(w[4 * q], xq.x, ha);
                                ha = fmaf(w[4 * q + 1], xq.y, ha);
                                ha = fmaf(w[4 * q + 2], xq.z, ha);
                                ha = fmaf(w[4 * q + 3], xq.w, ha);
                            }
                            hb = ha;
                        }
                        const LanePair hh = rows16(ha, hb);
                        s[pp][i] = (hh.lo + hh.hi) * dsf[i];
                    }
                }
#pragma unroll
                for (int pp = 0; pp < NPP; pp++) {
                    if (2 * pp >= nv) continue;
                    float t[CH > 1 ? CH / 2 : 1];
                    if constexpr (CH == 1) {
                        const LanePair vv = halves32(s[pp][0], s[pp][0]);
                        t[0] = 2 * g + 1 >= nb ? vv.lo : vv.lo + vv.hi;
                    } else {
#pragma unroll
                        for (int i = 0; i < CH / 2; i++) {
                            const LanePair vv = halves32(s[pp][i], s[pp][i + CH / 2]);
                            const int p = g * CH + i + (lane >= 32 ? CH / 2 : 0);
                            t[i] = p >= np ? -0.0f : 2 * p + 1 >= nb ? vv.lo : vv.lo + vv.hi;
                        }
#pragma unroll
                        for (int s2 = 1; s2 < CH / 2; s2 *= 2)
#pragma unroll
                            for (int i = 0; i + s2 < CH / 2; i += 2 * s2) t[i] = t[i] + t[i + s2];
                        const LanePair hl = halves32(t[0], t[0]);
                        t[0] = hl.lo + hl.hi;
                    }
                    if (lane < (2 * pp + 1 < nv ? 32 : 16))
                        gs[(((2 * pp + (lane >> 4)) * NT + tt) * G + g) * 16 + (lane & 15)] = t[0];
                }
            } else {
                // one vector per pass: each chunk's codes are unpacked as the
                // chain uses them (no unpacked copy held across chunks)
                for (int v = 0; v < nv; v++) {
                    const float* xv = xs + v * xstride;
                    float t[CH];
#pragma unroll
                    for (int i = 0; i < CH; i++) {
                        const int p = g * CH + i;  // past np: padding, skipped by the tree
                        const float h = dot16(cv[i], xv + (2 * p + bsel) * 32 + half * 16);
                        // h0 + h1 (half-0 lane's sum first) and v_2p + v_2p+1, v_2p alone
                        // when block 2p + 1 is the padding of an odd nb
                        const LanePair hh = lanes16(h);
                        const float vb = (hh.lo + hh.hi) * dsf[i];
                        const LanePair vv = lanes32(vb);
                        t[i] = 2 * p + 1 >= nb ? vv.lo : vv.lo + vv.hi;
                    }
#pragma unroll
                    for (int s = 1; s < CH; s *= 2)
#pragma unroll
                        for (int i = 0; i + s < CH; i += 2 * s)
                            if (i + s < cnt) t[i] = t[i] + t[i + s];
                    if (lane < 16) gs[((v * NT + tt) * G + g) * 16 + lane] = t[0];
                }
            }
        }
        __syncthreads();
        // ---- tree over the group sums, one thread per (vector, tile, row) ----
        if (tid < nv * NT * 16) {
            const int v = tid / (NT * 16), tt = (tid >> 4) % NT, rr = tid & 15;
            float* col = gs + (v * NT + tt) * G * 16 + rr;
            for (int s = 1; s < G; s *= 2)
                for (int i = 0; i + s < G; i += 2 * s) col[i * 16] = col[i * 16] + col[(i + s) * 16];
            if (EPI != EPI_SWIGLU) {
                const float acc = col[0];
                const int row = (tile + tt) * TILE_ROWS + rr;
                if (row < a.rows) {
                    const int ent = vbeg + v0 + v;
                    const int slot = a.slots ? a.slots[ent] : ent;
                    float* yp = a.y + (size_t)slot * a.y_stride + row;
                    if (EPI == EPI_RESID) *yp = a.resid[(size_t)slot * a.resid_stride + row] + acc;
                    else *yp = acc;
                }
            }
        }
        if (EPI == EPI_SWIGLU) {
            __syncthreads();
            if (tid < nv * 16) {
                // output row 8 tile + rr: gate row rr & 7 of tile tile + rr / 8, up row 8 + (rr & 7)
                const int v = tid >> 4, rr = tid & 15;
                const float* ts = gs + (v * NT + (rr >> 3)) * G * 16;
                const float gate = ts[rr & 7], up = ts[8 + (rr & 7)];
                const int row = tile * 8 + rr;  // < rows / 2 (a multiple of 16)
                const int ent = vbeg + v0 + v;
                const int slot = a.slots ? a.slots[ent] : ent;
                a.y[(size_t)slot * a.y_stride + row] = silu_mul(gate, up);
            }
        }
        __syncthreads();
    }
#undef MV_LOAD_ITEM
}

// Routed expert down projections of one token fused with their combine
// (batch 1): one workgroup per 16-row tile of the hidden state runs the GEMV
// of every routed expert over that tile -- the arithmetic of k_gemv_mv
// (16-code fmaf chains, the lane pair sums, the trees over a group's pairs
// and over the groups) -- then h[row] = h2[row] + sum over the experts in
// ascending index of w * y (k_moe_combine's order).  The expert outputs never
// leave the workgroup.
//
// FAST (K * G <= 32 items, G <= 8 groups, the inputs in 3 float4 per
// thread): the inputs -- which do not depend on the routing -- are loaded
// first, the routing (experts, weights) once per lane, then every item's
// weights (two per wave), so that no load waits behind another's round trip;
// the rank order comes from lane exchanges, and the trees over the groups
// and the combine run in registers of the first 16 lanes.  Otherwise the
// weights of a wave's next item are prefetched while it computes one.
constexpr int MOE_DOWN_THREADS = 1024;
constexpr int MOE_DOWN_FAST_GMAX = 8;

template <int CH, bool FAST>
__global__ __launch_bounds__(MOE_DOWN_THREADS) void k_moe_down_combine(MoeDownArgs a) {
    extern __shared__ float smem[];
    __shared__ int order[MOE_DOWN_MAX_K];
    __shared__ float ys[FAST ? MOE_DOWN_MAX_K * 16 : 1];  // FAST: rank q's outputs of the tile's rows
    constexpr int NW = MOE_DOWN_THREADS / 64;
    const int tile = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = a.K, k = a.k, k4 = k >> 2, nb = k >> 5, np = (nb + 1) >> 1;
    const int G = (np + CH - 1) / CH, items = K * G;
    float* xs = smem;                 // [K][np * 64]
    float* gs = xs + K * np * 64;     // [K][G][16]
    const int r = lane & 15, part = lane >> 4, bsel = part >> 1, half = part & 1;
    // group sum of item `it` = (rank-ordered expert q, group g) from its weights
    auto run_item = [&](int it, const u32x4 (&cv)[CH], const uint16_t (&ds)[CH]) {
        const int q = it / G, g = it - q * G;
        const float* xv = xs + q * np * 64;
        const int cnt = min(CH, np - g * CH);
        float t[CH];
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int p = min(g * CH + i, np - 1);
            u32x4 c = cv[i];
            // held items: the empty asm keeps the byte unpacking here
            if constexpr (FAST) asm volatile("" : "+v"(c.x), "+v"(c.y), "+v"(c.z), "+v"(c.w));
            const float h = dot16(c, xv + (2 * p + bsel) * 32 + half * 16);
            const LanePair hh = lanes16(h);
            const float vb = (hh.lo + hh.hi) * f16_bits_to_f32(ds[i]);
            const LanePair vv = lanes32(vb);
            t[i] = 2 * p + 1 >= nb ? vv.lo : vv.lo + vv.hi;
        }
#pragma unroll
        for (int s2 = 1; s2 < CH; s2 *= 2)
#pragma unroll
            for (int i = 0; i + s2 < CH; i += 2 * s2)
                if (i + s2 < cnt) t[i] = t[i] + t[i + s2];
        if (lane < 16) gs[(q * G + g) * 16 + lane] = t[0];
    };
    // weights of item `it`, clamped (every load in bounds), of expert e_of(q)
    auto load_item = [&](int it_, uint32_t e, u32x4 (&pv)[CH], uint16_t (&ps)[CH]) {
        const int itc = min(it_, items - 1), g = itc - (itc / G) * G;
        const size_t gt = (size_t)e * a.prob_tiles + tile;
        const int8_t* cb = a.codes + gt * np * CHUNK_BYTES + lane * 16;
        const uint16_t* sb = a.scales + gt * 2 * np * 16 + bsel * 16 + r;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int c = min(g * CH + i, np - 1);
            pv[i] = __builtin_nontemporal_load((const u32x4*)(cb + (size_t)c * CHUNK_BYTES));
            ps[i] = sb[(size_t)c * 32];
        }
    };
    if constexpr (FAST) {
        // the K inputs, entry i = q * k4 + i4 (clamped: every load in bounds)
        const int nx = K * k4;
        auto xaddr = [&](int i) {
            const int q = i / k4;
            return (const float4*)(a.x + (size_t)q * a.x_stride + 4 * (i - q * k4));
        };
        const float4 x0 = *xaddr(min(tid, nx - 1));
        const float4 x1 = *xaddr(min(tid + MOE_DOWN_THREADS, nx - 1));
        const float4 x2 = *xaddr(min(tid + 2 * MOE_DOWN_THREADS, nx - 1));
        // the routing: lane q holds rank q's expert and weight
        const uint32_t rid = a.rids[min(lane, K - 1)];
        const float rwt = a.rw[min(lane, K - 1)];
        const float h2 = a.h2[min(tile * TILE_ROWS + (lane & 15), a.rows - 1)];
        auto expert = [&](int it) {  // it wave-uniform
            const int q = min(it, items - 1) / G;
            return (uint32_t)__builtin_amdgcn_readlane((int)rid, q);
        };
        u32x4 pa[2][CH];
        uint16_t sa[2][CH];
        load_item(wave, expert(wave), pa[0], sa[0]);
        load_item(wave + NW, expert(wave + NW), pa[1], sa[1]);
        if (wave == 0 && lane < K) {
            int below = 0;
            for (int q = 0; q < K; q++) below += (uint32_t)__builtin_amdgcn_readlane((int)rid, q) < rid;
            order[below] = lane;  // the routed experts of a token are distinct
        }
        // stage the K input vectors in rank order (silu(gate) * up of each expert)
        auto xstore = [&](int i, float4 v) {
            if (i < nx) {
                const int q = i / k4;
                *(float4*)(xs + q * np * 64 + 4 * (i - q * k4)) = v;
            }
        };
        xstore(tid, x0);
        xstore(tid + MOE_DOWN_THREADS, x1);
        xstore(tid + 2 * MOE_DOWN_THREADS, x2);
        if (nb & 1)
            for (int i = tid; i < K * 32; i += MOE_DOWN_THREADS) xs[(i >> 5) * np * 64 + k + (i & 31)] = 0.0f;
        __syncthreads();
        if (wave < items) run_item(wave, pa[0], sa[0]);
        if (wave + NW < items) run_item(wave + NW, pa[1], sa[1]);
        __syncthreads();
        // the tree over each rank's groups, thread (rank, row) ...
        if (tid < K * 16) {
            float v[MOE_DOWN_FAST_GMAX];
#pragma unroll
            for (int i = 0; i < MOE_DOWN_FAST_GMAX; i++) v[i] = gs[((tid >> 4) * G + min(i, G - 1)) * 16 + (tid & 15)];
#pragma unroll
            for (int s2 = 1; s2 < MOE_DOWN_FAST_GMAX; s2 *= 2)
#pragma unroll
                for (int i = 0; i + s2 < MOE_DOWN_FAST_GMAX; i += 2 * s2)
                    if (i + s2 < G) v[i] = v[i] + v[i + s2];
            ys[tid] = v[0];
        }
        __syncthreads();
        // ... then the combine in ascending expert order (every LDS read issued at once)
        if (tid < 16) {
            int rk[MOE_DOWN_MAX_K];
            float y[MOE_DOWN_MAX_K];
#pragma unroll
            for (int qq = 0; qq < MOE_DOWN_MAX_K; qq++) rk[qq] = __builtin_amdgcn_readfirstlane(order[min(qq, K - 1)]);
#pragma unroll
            for (int qq = 0; qq < MOE_DOWN_MAX_K; qq++) y[qq] = ys[rk[qq] * 16 + tid];
            float acc = 0.0f;
#pragma unroll
            for (int qq = 0; qq < MOE_DOWN_MAX_K; qq++)
                if (qq < K) acc = acc + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rwt), rk[qq])) * y[qq];
            const int row = tile * TILE_ROWS + tid;
            if (row < a.rows) a.out[row] = h2 + acc;
        }
    } else {
        if (tid < K) {
            const uint32_t me = a.rids[tid];
            int below = 0;
            for (int q = 0; q < K; q++) below += a.rids[q] < me;
            order[below] = tid;  // the routed experts of a token are distinct
        }
        auto load = [&](int it_, u32x4 (&pv)[CH], uint16_t (&ps)[CH]) {
            load_item(it_, a.rids[min(it_, items - 1) / G], pv, ps);  // rank q's expert (raw rank order)
        };
        u32x4 pv[CH];
        uint16_t ps[CH];
        load(wave, pv, ps);
        // stage the K input vectors in rank order (silu(gate) * up of each expert)
        for (int q = 0; q < K; q++) {
            const float* x = a.x + (size_t)q * a.x_stride;
            float* xv = xs + q * np * 64;
            for (int i4 = tid; i4 < k4; i4 += MOE_DOWN_THREADS) *(float4*)(xv + 4 * i4) = *(const float4*)(x + 4 * i4);
            if ((nb & 1) && tid < 32) xv[k + tid] = 0.0f;
        }
        __syncthreads();
        for (int it = wave; it < items; it += NW) {
            u32x4 cv[CH];
            uint16_t ds[CH];
#pragma unroll
            for (int i = 0; i < CH; i++) {
                cv[i] = pv[i];
                ds[i] = ps[i];
            }
            load(it + NW, pv, ps);  // the next item's weights while this one computes
            run_item(it, cv, ds);
        }
        __syncthreads();
        // tree over the group sums, one thread per (rank, row)
        if (tid < K * 16) {
            float* col = gs + (tid >> 4) * G * 16 + (tid & 15);
            for (int s2 = 1; s2 < G; s2 *= 2)
                for (int i = 0; i + s2 < G; i += 2 * s2) col[i * 16] = col[i * 16] + col[(i + s2) * 16];
        }
        __syncthreads();
        if (tid < 16) {
            const int row = tile * TILE_ROWS + tid;
            float acc = 0.0f;
            for (int q = 0; q < K; q++) {
                const int rk = order[q];
                acc = acc + a.rw[rk] * gs[rk * G * 16 + tid];
            }
            if (row < a.rows) a.out[row] = a.h2[row] + acc;
        }
    }
}

// Routed expert gate and up projections of one token (batch 1) with the
// RMSNorm fused.  Every tile reads the same input and, the weight's tiles
// interleaving gate and up by 8 rows, gives silu(gate) * up of 8 rows by
// itself, so the K ranks' tiles (2 * inter / 16 of expert rids[q] each) form
// one list that the workgroups split evenly, GU1_TPW tiles each
// (Qwen3-30B-A3B: 768 tiles on 256 workgroups, one per compute unit); tile
// t of rank q stores rows 8t .. 8t+7 of y[q].  The arithmetic is k_gemv_mv's
// (XS_RMSNORM, EPI_SWIGLU): the SUM64 norm, 16-code fmaf chains, the lane
// pair sums, the trees over a group's pairs and over the groups.  Wave 0
// runs the norm alone: it loads the input and the norm weights (which do
// not depend on the routing), writes bf16(x) to LDS, reads it back in the
// SUM64 layout (one wave's LDS operations complete in order) and writes the
// normalised values.  Waves 1 .. 8 issue the weights of their (at most 3)
// items at once; their registers and the norm's are live in separate
// branches, so they do not add up, and their loads do not delay the norm
// wave's (spreading the norm over the item waves puts their weight loads
// ahead of it).  One barrier orders the input before the items, one the
// group sums before the trees over the groups, which run in registers.
constexpr int GU1_ITEM_WAVES = 8;
constexpr int GU1_AH = 3;                          // items per item wave
constexpr int GU1_TPW = 3;                         // tiles per workgroup
constexpr int GU1_THREADS = 64 * (1 + GU1_ITEM_WAVES);
constexpr int GU1_CH = 4;
constexpr int GU1_MAX_K = 2048;                    // the norm wave holds the input: 8 float4 per lane
constexpr int GU1_XF = GU1_MAX_K / 256;
constexpr int GU1_GMAX = GU1_MAX_K / 64 / GU1_CH;  // groups of a tile (np <= 32)
static_assert(GU1_TPW * GU1_GMAX <= GU1_ITEM_WAVES * GU1_AH, "a workgroup's items fit its item waves");
static_assert(GU1_TPW * 16 <= 64, "one wave runs the trees over the groups");

__global__ __launch_bounds__(GU1_THREADS) void k_moe_gate_up1(MoeGateUpArgs a) {
    extern __shared__ float smem[];
    constexpr int W = GU1_ITEM_WAVES, CH = GU1_CH;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ntt = a.K * a.prob_tiles, t0 = blockIdx.x * GU1_TPW, nt = min(GU1_TPW, ntt - t0);
    const int k = a.k, k4 = k >> 2, nb = k >> 5, np = (nb + 1) >> 1;
    const int G = (np + CH - 1) / CH, items = nt * G;
    float* xs = smem;               // [G * CH * 64]: the normed input, zero past k
    float* gs = xs + G * CH * 64;   // [GU1_TPW][G][16] group sums
    if (wave == 0) {
        float4 xv[GU1_XF], wv[GU1_XF];
#pragma unroll
        for (int j = 0; j < GU1_XF; j++) {
            const int i4 = min(lane + 64 * j, k4 - 1);
            xv[j] = *(const float4*)(a.x + 4 * i4);
            wv[j] = *(const float4*)(a.norm_w + 4 * i4);
        }
        // RmsNorm (src/rms_norm.rs:143-176): v = bf16(x); the sum of squares in
        // the SUM64 order; inv = 1 / sqrt(sum / k + eps); n = bf16((v * inv) * bf16(w))
#pragma unroll
        for (int j = 0; j < GU1_XF; j++)
            if (lane + 64 * j < k4) *(float4*)(xs + 4 * (lane + 64 * j)) = bf16_round4(xv[j]);
        float v[GU1_MAX_K / 64];
#pragma unroll
        for (int u = 0; u < GU1_MAX_K / 64; u++) v[u] = xs[min(lane + 64 * u, k - 1)];
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < GU1_MAX_K / 64; u++)
            if (lane + 64 * u < k) acc = acc + v[u] * v[u];
        acc = wave_sum64(acc);
        const float inv = __fdiv_rn(1.0f, __builtin_sqrtf(__fdiv_rn(acc, (float)k) + a.eps));
#pragma unroll
        for (int j = 0; j < GU1_XF; j++)
            if (lane + 64 * j < k4) {
                float4* p = (float4*)(xs + 4 * (lane + 64 * j));
                *p = norm4(*p, wv[j], inv);  // bf16(x) read back: xv is not held across the sum
            }
        // the group padding past k (read by the padding pairs, never summed)
        for (int i = k + lane; i < G * CH * 64; i += 64) xs[i] = 0.0f;
        __syncthreads();
    } else {
        const int r = lane & 15, part = lane >> 4, bsel = part >> 1, half = part & 1;
        const int w = wave - 1;
        const uint32_t rid = a.rids[min(lane, a.K - 1)];  // lane q: rank q's expert
        // the weights of this wave's items (clamped: every load in bounds)
        u32x4 pa[GU1_AH][CH];
        uint16_t sa[GU1_AH][CH];
#pragma unroll
        for (int jj = 0; jj < GU1_AH; jj++) {
            const int it = min(w + W * jj, items - 1), tt = it / G, g = it - tt * G;
            const int q = (t0 + tt) / a.prob_tiles, lt = t0 + tt - q * a.prob_tiles;
            const size_t gt = (size_t)(uint32_t)__builtin_amdgcn_readlane((int)rid, q) * a.prob_tiles + lt;
            const int8_t* cb = a.codes + gt * np * CHUNK_BYTES + lane * 16;
            const uint16_t* sb = a.scales + gt * 2 * np * 16 + bsel * 16 + r;
#pragma unroll
            for (int i = 0; i < CH; i++) {
                const int c = min(g * CH + i, np - 1);
                pa[jj][i] = __builtin_nontemporal_load((const u32x4*)(cb + (size_t)c * CHUNK_BYTES));
                sa[jj][i] = sb[(size_t)c * 32];
            }
        }
        __syncthreads();
#pragma unroll
        for (int jj = 0; jj < GU1_AH; jj++) {
            const int it = w + W * jj;
            if (it < items) {
                const int tt = it / G, g = it - tt * G;
                const int cnt = min(CH, np - g * CH);
                float t[CH];
#pragma unroll
                for (int i = 0; i < CH; i++) {
                    const int p = g * CH + i;  // past np: padding, skipped by the tree
                    u32x4 c = pa[jj][i];
                    asm volatile("" : "+v"(c.x), "+v"(c.y), "+v"(c.z), "+v"(c.w));  // unpack here, not at the load
                    const float h = dot16(c, xs + (2 * p + bsel) * 32 + half * 16);
                    // h0 + h1 (half-0 lane's sum first) and v_2p + v_2p+1, v_2p alone
                    // when block 2p + 1 is the padding of an odd nb
                    const LanePair hh = lanes16(h);
                    const float vb = (hh.lo + hh.hi) * f16_bits_to_f32(sa[jj][i]);
                    const LanePair vv = lanes32(vb);
                    t[i] = 2 * p + 1 >= nb ? vv.lo : vv.lo + vv.hi;
                }
#pragma unroll
                for (int s2 = 1; s2 < CH; s2 *= 2)
#pragma unroll
                    for (int i = 0; i + s2 < CH; i += 2 * s2)
                        if (i + s2 < cnt) t[i] = t[i] + t[i + s2];
                if (lane < 16) gs[(tt * G + g) * 16 + lane] = t[0];
            }
        }
    }
    __syncthreads();
    if (wave == 0) {
        // the tree over a tile's groups: lane (tile tt, row rr); the 16 lanes
        // of a tile hold its 8 gate rows, then its 8 up rows
        const int tt = min(lane >> 4, nt - 1), rr = lane & 15;
        float v[GU1_GMAX];
#pragma unroll
        for (int i = 0; i < GU1_GMAX; i++) v[i] = gs[(tt * G + min(i, G - 1)) * 16 + rr];
#pragma unroll
        for (int s2 = 1; s2 < GU1_GMAX; s2 *= 2)
#pragma unroll
            for (int i = 0; i + s2 < GU1_GMAX; i += 2 * s2)
                if (i + s2 < G) v[i] = v[i] + v[i + s2];
        const float up = lane_xor<8>(v[0]);
        const int q = (t0 + tt) / a.prob_tiles, lt = t0 + tt - q * a.prob_tiles;
        if (lane < nt * 16 && rr < 8) a.y[(size_t)q * a.y_stride + lt * 8 + rr] = silu_mul(v[0], up);
    }
}

// Greedy pick (src/generate.rs:153-174 via src/tensor.rs:2451-2480):
// maximum over the tiles' partials, last index on ties.
__global__ __launch_bounds__(1024) void k_argmax_final(const float* __restrict__ val, const int* __restrict__ idx,
                                                       int count, uint32_t* d_tok, uint32_t* tokens_out, int* d_pos,
                                                       int* d_step) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -__builtin_huge_valf();
    int bi = -1;
    constexpr int AU = 16;  // entries per thread per pass, loads issued together
    for (int i0 = tid; i0 < count; i0 += 1024 * AU) {
        float v[AU];
        int j[AU];
#pragma unroll
        for (int e = 0; e < AU; e++) {
            const int i = min(i0 + e * 1024, count - 1);
            v[e] = val[i];
            j[e] = idx[i];
        }
#pragma unroll
        for (int e = 0; e < AU; e++)
            if (i0 + e * 1024 < count && (v[e] > bv || (v[e] == bv && j[e] > bi))) { bv = v[e]; bi = j[e]; }
    }
    argmax_step<32>(bv, bi);
    argmax_step<16>(bv, bi);
    argmax_step<8>(bv, bi);
    argmax_step<4>(bv, bi);
    argmax_step<2>(bv, bi);
    argmax_step<1>(bv, bi);
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++)
            if (sv[w] > bv || (sv[w] == bv && si[w] > bi)) { bv = sv[w]; bi = si[w]; }
        const uint32_t tok = (uint32_t)(bi < 0 ? 0 : bi);
        *d_tok = tok;
        tokens_out[*d_step] = tok;
        *d_step = *d_step + 1;
        *d_pos = *d_pos + 1;
    }
}

constexpr int MANY_TILES = 512;  // 16-row tiles from which a GEMV takes the many-tiles launch shape

template <int XS, int EPI>
lq8_status launch_one(hipStream_t s, const GemvArgs& a) {
    const int nb = a.k >> 5, npf = (nb + 1) >> 1;
    // EPI_PART: a workgroup stages one chunk of part_pairs pairs
    const int np = EPI == EPI_PART ? std::min(npf, a.part_pairs) : npf;
    const int nch = EPI == EPI_PART ? (npf + a.part_pairs - 1) / a.part_pairs : 1;
    const int tiles = (a.n + TILE_ROWS - 1) / TILE_ROWS;
    // Many tiles (lm_head, and from two per CU: MANY_TILES): 4 pairs per
    // item, 4-wave workgroups with the next item's weights prefetched; a plain
    // input takes one tile per workgroup, a transformed one (RMSNorm) is
    // staged once for 2 tiles (151936 x 1024: 26.8 / 27.9 / 29.2 us plain and
    // 1246 / 1248 / 1244 decode tok/s at 1 / 2 / 4 tiles).  Few tiles: one
    // tile per workgroup and up to 16 waves to spread it over the CU.  The
    // boundary, measured on greedy decode: Qwen3-1.7B's gate|up (768 tiles)
    // 1036 -> 1079 tok/s as many, Qwen3-4B's q|k|v (384 tiles, K 2560) 575 ->
    // 565 and its gate|up (1216 tiles) 575 -> 519 as few.
    int ch, tpw, waves;
    const int wmax = tiles >= MANY_TILES ? 4 : MAX_WAVES;
    if (tiles >= MANY_TILES) {
        ch = MAX_CH;
        tpw = XS == XS_PLAIN ? 1 : 2;
    } else {
        ch = pick_ch(np, MAX_WAVES);
        tpw = 1;
    }
    const int G = (np + ch - 1) / ch;
    waves = max(tpw, min(wmax, tpw * G));
    size_t smem = ((size_t)np * 64 + (size_t)tpw * G * 16 + 4) * sizeof(float);
    if (XS == XS_ATTN)
        smem += ((size_t)std::min(a.attn_cmax, ATT_CB) * a.attn_heads * 2 + (1 + CU) * a.attn_heads) * sizeof(float);
    if (smem > 64 * 1024) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: input staging exceeds 64 KiB of LDS");
    const dim3 grid((unsigned)((tiles + tpw - 1) / tpw), (unsigned)nch), block(64 * waves);
    if (ch == 1) hipLaunchKernelGGL((k_gemv<XS, EPI, 1>), grid, block, smem, s, a, tpw);
    else if (ch == 2) hipLaunchKernelGGL((k_gemv<XS, EPI, 2>), grid, block, smem, s, a, tpw);
    else hipLaunchKernelGGL((k_gemv<XS, EPI, 4>), grid, block, smem, s, a, tpw);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

template <int XS>
lq8_status launch_epi(hipStream_t s, Epilogue epi, const GemvArgs& a) {
    switch (epi) {
        case EPI_STORE: return launch_one<XS, EPI_STORE>(s, a);
        case EPI_RESID: return launch_one<XS, EPI_RESID>(s, a);
        default: return launch_one<XS, EPI_ARGMAX>(s, a);
    }
}

}  // namespace

lq8_status launch_gemv(hipStream_t s, XSource xs, Epilogue epi, const GemvArgs& a) {
    if (a.k <= 0 || a.k % 32 || a.n <= 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k must be a positive multiple of 32");
    if (a.k > GEMV_MAX_K) {
        // a plain input streams through LDS in stages; the fused inputs need the whole vector staged
        if (xs != XS_PLAIN || epi != EPI_STORE)
            return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k above 12288 is supported for a plain input only");
        if (a.k > GEMV_LONG_MAX_K) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k above 131072 is not supported");
        const int np = ((a.k >> 5) + 1) >> 1, G = (np + LONG_CH - 1) / LONG_CH;
        const size_t smem = ((size_t)LONG_PAIRS * 64 + (size_t)G * 16) * sizeof(float);
        const dim3 grid((unsigned)((a.n + TILE_ROWS - 1) / TILE_ROWS));
        hipLaunchKernelGGL(k_gemv_long, grid, dim3(LONG_THREADS), smem, s, a);
        LQ8_HIP(hipGetLastError());
        return LQ8_OK;
    }
    if (epi == EPI_RESID && !a.resid) return fail(LQ8_ERR_INVALID_ARG, "gemv: residual is null");
    if (epi == EPI_ARGMAX && (!a.arg_val || !a.arg_idx)) return fail(LQ8_ERR_INVALID_ARG, "gemv: argmax buffers are null");
    if (xs == XS_ATTN && (a.attn_heads * 128 != a.k || a.attn_cmax <= 0))
        return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: attention input layout does not match k");
    if (xs == XS_SILU_PART || epi == EPI_PART) {
        const int pp = a.part_pairs;
        if (xs != XS_SILU_PART || epi != EPI_PART || pp <= 0 || (pp & (pp - 1)))
            return fail(LQ8_ERR_INVALID_ARG, "gemv: input chunks need the chunked silu input and a power-of-two pair count");
        return launch_one<XS_SILU_PART, EPI_PART>(s, a);
    }
    if (xs == XS_RMSNORM_JOIN) {
        if (!a.parts || a.nparts < 1 || a.nparts > 4 || !a.h_out || !a.norm_w)
            return fail(LQ8_ERR_INVALID_ARG, "gemv: the join needs 1 to 4 chunk-sum vectors, h_out and the norm weight");
        if (epi == EPI_STORE) return launch_one<XS_RMSNORM_JOIN, EPI_STORE>(s, a);
        if (epi == EPI_ARGMAX) return launch_one<XS_RMSNORM_JOIN, EPI_ARGMAX>(s, a);
        return fail(LQ8_ERR_INVALID_ARG, "gemv: the join stages a plain or argmax GEMV only");
    }
    switch (xs) {
        case XS_PLAIN: return launch_epi<XS_PLAIN>(s, epi, a);
        case XS_RMSNORM: return launch_epi<XS_RMSNORM>(s, epi, a);
        case XS_SILU: return launch_epi<XS_SILU>(s, epi, a);
        default: return launch_epi<XS_ATTN>(s, epi, a);
    }
}

lq8_status launch_gemv_grouped(hipStream_t s, const GemvProblemDev* d_probs, int count, int total_tiles,
                               int max_k) {
    if (count <= 0 || total_tiles <= 0) return LQ8_OK;
    // throughput form: 4 waves per tile, 4 pairs per group (a wave loops over groups)
    const int np = ((max_k >> 5) + 1) >> 1;
    const int gmax = (np + MAX_CH - 1) / MAX_CH;
    const size_t smem = ((size_t)np * 64 + (size_t)gmax * 16 + 4) * sizeof(float);
    hipLaunchKernelGGL(k_gemv_grouped, dim3((unsigned)total_tiles), dim3(256), smem, s, d_probs, count);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

namespace {

template <int XS, int EPI, int CH, int NTS>
lq8_status mv_vb(hipStream_t s, const MvArgs& a, dim3 grid, int vb, size_t xs_floats_per_vec, int G) {
    const size_t NT = EPI == EPI_SWIGLU ? 2 : NTS;
    const size_t smem = ((size_t)vb * xs_floats_per_vec + (size_t)vb * NT * G * 16 + 4) * sizeof(float);
    if (smem > 64 * 1024) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: input staging exceeds 64 KiB of LDS");
    // single vector and more items than waves: the pipelined variant (with
    // several vectors the prefetch registers cost more occupancy than it hides)
    if (a.max_vec == 1 && NT * G > 4)
        hipLaunchKernelGGL((k_gemv_mv<XS, EPI, CH, 1, true, NTS>), grid, dim3(256), smem, s, a);
    else if (vb == 4) hipLaunchKernelGGL((k_gemv_mv<XS, EPI, CH, 4, false, NTS>), grid, dim3(256), smem, s, a);
    else if (vb == 2) hipLaunchKernelGGL((k_gemv_mv<XS, EPI, CH, 2, false, NTS>), grid, dim3(256), smem, s, a);
    else hipLaunchKernelGGL((k_gemv_mv<XS, EPI, CH, 1, false, NTS>), grid, dim3(256), smem, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

template <int XS, int EPI, int NTS>
lq8_status mv_nts(hipStream_t s, const MvArgs& a, int max_probs, int vsplit) {
    const int nb = a.k >> 5, np = (nb + 1) >> 1;
    const int ch = pick_ch(np, 4);
    const int G = (np + ch - 1) / ch;
    const size_t per_vec = (size_t)G * ch * 64;  // np pairs padded to whole groups
    // vectors staged per pass: as many as fit in 40 KiB
    int vb = per_vec * 4 * sizeof(float) <= 40 * 1024 ? 4 : per_vec * 2 * sizeof(float) <= 40 * 1024 ? 2 : 1;
    if (a.max_vec == 1 && (EPI == EPI_SWIGLU ? 2 : NTS) * G > 4) vb = 1;  // the pipelined variant stages one vector
    const int tiles_p = (a.rows + TILE_ROWS - 1) / TILE_ROWS / (EPI == EPI_SWIGLU ? 2 : NTS);
    const dim3 grid((unsigned)(tiles_p * max_probs), (unsigned)vsplit);
    if (ch == 1) return mv_vb<XS, EPI, 1, NTS>(s, a, grid, vb, per_vec, G);
    if (ch == 2) return mv_vb<XS, EPI, 2, NTS>(s, a, grid, vb, per_vec, G);
    return mv_vb<XS, EPI, 4, NTS>(s, a, grid, vb, per_vec, G);
}

template <int XS, int EPI>
lq8_status mv_ch(hipStream_t s, const MvArgs& a, int max_probs, int vsplit) {
    if constexpr (XS == XS_PLAIN && EPI == EPI_STORE) {
        // routed problem lists of several vectors (the experts' down
        // projections at batch > 1): 4 consecutive tiles per workgroup, the
        // inputs staged once for all of them
        const int tiles_all = (a.rows + TILE_ROWS - 1) / TILE_ROWS;
        if (max_probs > 1 && a.max_vec > 1 && tiles_all % 4 == 0) return mv_nts<XS, EPI, 4>(s, a, max_probs, vsplit);
    }
    return mv_nts<XS, EPI, 1>(s, a, max_probs, vsplit);
}

}  // namespace

lq8_status launch_gemv_mv(hipStream_t s, XSource xs, Epilogue epi, const MvArgs& a, int max_probs, int vsplit) {
    if (a.k <= 0 || a.k % 32 || a.rows <= 0) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k must be a positive multiple of 32");
    if (a.k > GEMV_MAX_K) return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: k above 12288 is not supported");
    if (max_probs <= 0 || vsplit <= 0) return LQ8_OK;
    if (epi == EPI_RESID && !a.resid) return fail(LQ8_ERR_INVALID_ARG, "gemv: residual is null");
    if (xs == XS_RMSNORM && !a.norm_w) return fail(LQ8_ERR_INVALID_ARG, "gemv: norm weight is null");
    if (epi == EPI_ARGMAX || xs == XS_ATTN) return fail(LQ8_ERR_INVALID_ARG, "gemv: unsupported multi-vector mode");
    if (a.x_div <= 0) return fail(LQ8_ERR_INVALID_ARG, "gemv: x_div must be positive");
    if (epi == EPI_SWIGLU) {
        if (a.rows % (2 * TILE_ROWS) || (xs != XS_RMSNORM && xs != XS_PLAIN))
            return fail(LQ8_ERR_SHAPE_MISMATCH, "gemv: swiglu needs rows a multiple of 32 and a plain or normed input");
        return xs == XS_PLAIN ? mv_ch<XS_PLAIN, EPI_SWIGLU>(s, a, max_probs, vsplit)
                              : mv_ch<XS_RMSNORM, EPI_SWIGLU>(s, a, max_probs, vsplit);
    }
    const bool resid = epi == EPI_RESID;
    switch (xs) {
        case XS_PLAIN: return resid ? mv_ch<XS_PLAIN, EPI_RESID>(s, a, max_probs, vsplit)
                                    : mv_ch<XS_PLAIN, EPI_STORE>(s, a, max_probs, vsplit);
        case XS_RMSNORM: return resid ? mv_ch<XS_RMSNORM, EPI_RESID>(s, a, max_probs, vsplit)
                                      : mv_ch<XS_RMSNORM, EPI_STORE>(s, a, max_probs, vsplit);
        default: return resid ? mv_ch<XS_SILU, EPI_RESID>(s, a, max_probs, vsplit)
                              : mv_ch<XS_SILU, EPI_STORE>(s, a, max_probs, vsplit);
    }
}

bool moe_down_combine_supported(int K, int k) {
    const int nb = k >> 5, np = (nb + 1) >> 1, ch = pick_ch(np, 4), G = (np + ch - 1) / ch;
    const size_t smem = ((size_t)K * np * 64 + (size_t)K * G * 16) * sizeof(float);
    return K >= 1 && K <= MOE_DOWN_MAX_K && k > 0 && k % 32 == 0 && smem <= 48 * 1024;
}

lq8_status launch_moe_down_combine(hipStream_t s, const MoeDownArgs& a) {
    if (!moe_down_combine_supported(a.K, a.k) || a.rows <= 0 || a.rows % TILE_ROWS)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe down+combine: unsupported shape");
    const int nb = a.k >> 5, np = (nb + 1) >> 1, ch = pick_ch(np, 4), G = (np + ch - 1) / ch;
    const size_t smem = ((size_t)a.K * np * 64 + (size_t)a.K * G * 16) * sizeof(float);
    const dim3 grid((unsigned)(a.rows / TILE_ROWS));
    // every item's weights in flight at once (two items per wave), the inputs in registers
    const bool fast = ch == 4 && a.K * G <= 2 * (MOE_DOWN_THREADS / 64) && G <= MOE_DOWN_FAST_GMAX &&
                      a.K * (a.k >> 2) <= 3 * MOE_DOWN_THREADS && a.K <= 64;
    const dim3 block(MOE_DOWN_THREADS);
    if (fast) hipLaunchKernelGGL((k_moe_down_combine<4, true>), grid, block, smem, s, a);
    else if (ch == 1) hipLaunchKernelGGL((k_moe_down_combine<1, false>), grid, block, smem, s, a);
    else if (ch == 2) hipLaunchKernelGGL((k_moe_down_combine<2, false>), grid, block, smem, s, a);
    else hipLaunchKernelGGL((k_moe_down_combine<4, false>), grid, block, smem, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

bool moe_gate_up1_supported(int K, int inter, int k) {
    return K >= 1 && K <= 64 && inter > 0 && inter % TILE_ROWS == 0 && k > 0 && k % 32 == 0 && k <= GU1_MAX_K;
}

lq8_status launch_moe_gate_up1(hipStream_t s, const MoeGateUpArgs& a) {
    if (!moe_gate_up1_supported(a.K, a.inter, a.k) || a.prob_tiles != 2 * a.inter / TILE_ROWS ||
        a.y_stride < a.inter)
        return fail(LQ8_ERR_SHAPE_MISMATCH, "moe gate+up: unsupported shape");
    const int nb = a.k >> 5, np = (nb + 1) >> 1, G = (np + GU1_CH - 1) / GU1_CH;
    const size_t smem = ((size_t)G * GU1_CH * 64 + (size_t)GU1_TPW * G * 16) * sizeof(float);
    const dim3 grid((unsigned)((a.K * a.prob_tiles + GU1_TPW - 1) / GU1_TPW));
    hipLaunchKernelGGL(k_moe_gate_up1, grid, dim3(GU1_THREADS), smem, s, a);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

lq8_status launch_argmax_final(hipStream_t s, const float* arg_val, const int* arg_idx, int count, uint32_t* d_tok,
                               uint32_t* tokens_out, int* d_pos, int* d_step) {
    if (count <= 0) return fail(LQ8_ERR_INVALID_ARG, "argmax: empty");
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(1024), 0, s, arg_val, arg_idx, count, d_tok, tokens_out, d_pos,
                       d_step);
    LQ8_HIP(hipGetLastError());
    return LQ8_OK;
}

}  // namespace lq8
