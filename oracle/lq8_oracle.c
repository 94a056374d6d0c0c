/*
 * lq8_oracle.c -- CPU oracle for the Q8_0 quantized-weight hot path of
 * lluda-inference (TEST INFRASTRUCTURE: loaded only by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg, always as the
 * checker, never as the thing shipped or measured as the product).
 *
 * What it restates
 *   - Q8_0 (GGUF block_q8_0: f16 scale + 32 int8 codes, 34 bytes) quantize /
 *     dequantize.  The reference names this format as its plan
 *     (README.md:24,32; docs/architecture/arch-2026-01-31-qwen3-omni-q8-rust.md:36-39,275-279)
 *     and places the arithmetic in candle-core's GGML quantized module
 *     (arch-2026-01-31-qwen3-bf16-first.md:309-315), which is not vendored.
 *     Published algorithm restated: amax = max|x| (NaN ignored, as f32::max),
 *     d = amax/127, id = d ? 1/d : 0, q = round_half_away(x*id) saturated to
 *     int8 (NaN -> 0), scale stored as f16 (round to nearest even).
 *   - Linear::forward (lluda-inference/src/attention.rs:101-136) on a Q8_0
 *     weight: y[m, n] = x[m, :] . W[n, :].  M == 1 is a W8A32 GEMV, M > 1
 *     quantizes the activation rows and runs a W8A8 GEMM with exact int32 per
 *     block and an f32 rescale.
 *   - The Qwen3 decoder numerics around it: RmsNorm (src/rms_norm.rs:123-177,
 *     bf16 input and output rounding), RoPE (src/rope.rs:77-128,245-303),
 *     GQA attention (src/attention.rs:318-403, 426-456), softmax
 *     (src/tensor.rs:1913-1935), SiLU (src/tensor.rs:1955-1990), residual adds
 *     (src/transformer.rs:180-204), last-token lm_head (src/model.rs:345-372),
 *     greedy argmax with last-index ties (src/tensor.rs:2451-2480,
 *     src/generate.rs:153-174, 611-664).
 *
 * Canonical orders (the HIP kernels follow exactly these, so results match
 * bit for bit; the reference's own sums are plain sequential loops, available
 * here through orc_set_sequential_sums(1) for comparison):
 *   GEMV   per row: for block b, h0_b = fmaf chain over codes j = 0..15 and
 *          h1_b = fmaf chain over codes j = 16..31 (each from +0, in j order),
 *          v_b = (h0_b + h1_b) * d_b; then a pairwise tree over the blocks:
 *          for s = 1, 2, 4, ...: v[i] = v[i] + v[i + s] for i = 0, 2s, 4s, ...
 *          while i + s < nb; y = v[0].
 *   GEMM   per (m, n): I_b = exact int32 sum of the 32 code products;
 *          s_b = f32(dw_b) * f32(dx_b) (exact); a_g = fmaf((float)I_b, s_b, a_g)
 *          within a group of 8 blocks; y = y + a_g in group order.
 *   SUM64  (RMSNorm sum of squares, softmax denominator): lane l in 0..63
 *          accumulates elements l, l+64, l+128, ... in order from 0; then the
 *          64 partials are folded with distances 32, 16, 8, 4, 2, 1
 *          (v[l] = v[l] + v[l+d]).
 *   q.k     sequential over head_dim, as the reference's matmul_4d
 *          (src/tensor.rs:2846-2915).
 *   ATTN   softmax and p.v over segments of 64 positions with a running
 *          max / denominator (see attend()).
 *   exp    orc_expf: double-precision Cody-Waite reduction + degree-13 Taylor
 *          polynomial, rounded once to float.  Agrees with a correctly rounded
 *          expf except in rare last-bit cases; orc_set_libm_exp(1) uses the C
 *          library's expf instead (the reference's f32::exp on linux-gnu).
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math (Rust never contracts a*b+c).
 */
#include "lq8_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_seq_sums = 0;
void orc_set_sequential_sums(int on) { g_seq_sums = on ? 1 : 0; }

/* 1: the decoder's exp (attention softmax, SiLU) is the host C library's
 * expf -- on linux-gnu glibc's, the function Rust's f32::exp calls there, so
 * together with the sequential sums this is the reference's own arithmetic.
 * 0 (default): orc_expf, the exp the HIP kernels reproduce bit for bit. */
static int g_libm_exp = 0;
void orc_set_libm_exp(int on) { g_libm_exp = on ? 1 : 0; }

/* 1 (default): RmsNorm rounds its input, weight and output to bf16 as the
 * reference does.  0: those roundings are skipped.  Used only by the tests
 * that pin the decoder's structure against a float64 restatement, where a
 * bf16 rounding that lands on the other side of a midpoint (an f32-vs-f64
 * difference of one ulp) would otherwise hide everything else. */
static int g_bf16_sites = 1;
void orc_set_bf16_rounding(int on) { g_bf16_sites = on ? 1 : 0; }
static inline float site_bf16(float x) { return g_bf16_sites ? orc_bf16_round(x) : x; }

/* Thread count of the parallel loops (each output is still summed by one
 * thread in the fixed order, so results do not depend on it). */
void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------------------------ */
/* scalar numerics                                                          */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16, round to nearest even, with subnormals, overflow to inf. */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {
        if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 */
    if (ax >= 0x38800000u) {                                   /* >= 2^-14: normal */
        uint32_t mant = ax & 0x7FFFFFu;
        uint32_t e = (ax >> 23) - 127u + 15u;
        uint32_t h = (e << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 */
    {
        uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        int e = (int)(ax >> 23) - 127; /* -25 .. -15 */
        int s = -e - 1;                /* 14 .. 24 */
        uint32_t h = mant >> s;
        uint32_t rem = mant & ((1u << s) - 1u);
        uint32_t half = 1u << (s - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        /* subnormal or zero: m * 2^-24, exact in f32 */
        float v = (float)m * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* src/bf16.rs:112-131: bits + 0x7FFF + lsb, keep the top 16 bits. */
float orc_bf16_round(float x) {
    uint32_t b = f2u(x);
    uint32_t bias = 0x7FFFu + ((b >> 16) & 1u);
    return u2f(((b + bias) >> 16) << 16);
}

/* exp in double, rounded once to float.  Every step is an IEEE operation
 * (fma, mul, add, rint, ldexp), so any IEEE machine gets the same bits. */
float orc_expf(float xf) {
    if (xf != xf) return xf;
    if (xf > 89.0f) return INFINITY;
    if (xf < -110.0f) return 0.0f;
    double x = (double)xf;
    double k = rint(x * 1.4426950408889634074);
    double r = fma(-k, 6.93147180369123816490e-01, x);  /* ln2 hi */
    r = fma(-k, 1.90821492927058770002e-10, r);         /* ln2 lo */
    double p = 1.0 / 6227020800.0;                       /* 1/13! */
    p = fma(p, r, 1.0 / 479001600.0);
    p = fma(p, r, 1.0 / 39916800.0);
    p = fma(p, r, 1.0 / 3628800.0);
    p = fma(p, r, 1.0 / 362880.0);
    p = fma(p, r, 1.0 / 40320.0);
    p = fma(p, r, 1.0 / 5040.0);
    p = fma(p, r, 1.0 / 720.0);
    p = fma(p, r, 1.0 / 120.0);
    p = fma(p, r, 1.0 / 24.0);
    p = fma(p, r, 1.0 / 6.0);
    p = fma(p, r, 0.5);
    p = fma(p, r, 1.0);
    p = fma(p, r, 1.0);
    return (float)ldexp(p, (int)k);
}

void orc_f32_to_f16_n(const float* x, uint16_t* h, size_t n) { for (size_t i = 0; i < n; i++) h[i] = orc_f32_to_f16(x[i]); }
void orc_f16_to_f32_n(const uint16_t* h, float* x, size_t n) { for (size_t i = 0; i < n; i++) x[i] = orc_f16_to_f32(h[i]); }
void orc_bf16_round_n(const float* x, float* y, size_t n) { for (size_t i = 0; i < n; i++) y[i] = orc_bf16_round(x[i]); }
void orc_expf_n(const float* x, float* y, size_t n) { for (size_t i = 0; i < n; i++) y[i] = orc_expf(x[i]); }

/* SUM64 canonical order over v[0..n) (see header comment). */
static float sum64(const float* v, size_t n) {
    if (g_seq_sums) {
        float s = 0.0f;
        for (size_t i = 0; i < n; i++) s = s + v[i];
        return s;
    }
    float p[64];
    for (int l = 0; l < 64; l++) {
        float a = 0.0f;
        for (size_t i = (size_t)l; i < n; i += 64) a = a + v[i];
        p[l] = a;
    }
    for (int d = 32; d >= 1; d >>= 1)
        for (int l = 0; l < d; l++) p[l] = p[l] + p[l + d];
    return p[0];
}

/* ------------------------------------------------------------------------ */
/* Q8_0 format                                                              */
/* ------------------------------------------------------------------------ */

static inline int8_t sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

static void quantize_block(const float* x, uint16_t* d16, int8_t* q, float* d32) {
    float amax = 0.0f;
    for (int j = 0; j < ORC_QK; j++) {
        float v = fabsf(x[j]);
        if (v > amax) amax = v;
    }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    *d16 = orc_f32_to_f16(d);
    if (d32) *d32 = d;
    for (int j = 0; j < ORC_QK; j++) q[j] = sat_i8(roundf(x[j] * id));
}

int orc_quantize_q8_0(const float* x, size_t n, uint8_t* blocks) {
    if (n % ORC_QK) return 1;
    for (size_t b = 0; b < n / ORC_QK; b++) {
        uint16_t d16;
        int8_t q[ORC_QK];
        quantize_block(x + b * ORC_QK, &d16, q, NULL);
        uint8_t* o = blocks + b * ORC_BLOCK_BYTES;
        o[0] = (uint8_t)(d16 & 0xFF);
        o[1] = (uint8_t)(d16 >> 8);
        memcpy(o + 2, q, ORC_QK);
    }
    return 0;
}

static inline float blk_scale(const uint8_t* blk) {
    return orc_f16_to_f32((uint16_t)(blk[0] | ((uint16_t)blk[1] << 8)));
}

int orc_dequantize_q8_0(const uint8_t* blocks, size_t n, float* y) {
    if (n % ORC_QK) return 1;
    for (size_t b = 0; b < n / ORC_QK; b++) {
        const uint8_t* blk = blocks + b * ORC_BLOCK_BYTES;
        float d = blk_scale(blk);
        const int8_t* q = (const int8_t*)(blk + 2);
        for (int j = 0; j < ORC_QK; j++) y[b * ORC_QK + j] = d * (float)q[j];
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Q8_0 GEMV (W8A32) and GEMM (W8A8)                                        */
/* ------------------------------------------------------------------------ */

#define ORC_MAX_NB 4096 /* k_in <= 131072 */

/* GEMV canonical order (header comment); v is scratch of nb floats. */
static float gemv_row(const uint8_t* row, size_t nb, const float* x, float* v) {
    if (g_seq_sums) {
        /* matmul_2d (src/tensor.rs:2740-2750) over the dequantized row */
        float s = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t* blk = row + b * ORC_BLOCK_BYTES;
            float d = blk_scale(blk);
            const int8_t* q = (const int8_t*)(blk + 2);
            for (int j = 0; j < ORC_QK; j++) s = s + (d * (float)q[j]) * x[b * ORC_QK + j];
        }
        return s;
    }
    for (size_t b = 0; b < nb; b++) {
        const uint8_t* blk = row + b * ORC_BLOCK_BYTES;
        const int8_t* q = (const int8_t*)(blk + 2);
        const float* xb = x + b * ORC_QK;
        float h0 = 0.0f, h1 = 0.0f;
        for (int j = 0; j < 16; j++) h0 = fmaf((float)q[j], xb[j], h0);
        for (int j = 16; j < 32; j++) h1 = fmaf((float)q[j], xb[j], h1);
        v[b] = (h0 + h1) * blk_scale(blk);
    }
    for (size_t s = 1; s < nb; s *= 2)
        for (size_t i = 0; i + s < nb; i += 2 * s) v[i] = v[i] + v[i + s];
    return v[0];
}

int orc_gemv_q8_0(const uint8_t* w, size_t n_out, size_t k_in, const float* x, float* y) {
    if (k_in == 0 || k_in % ORC_QK || n_out == 0 || k_in / ORC_QK > ORC_MAX_NB) return 1;
    size_t nb = k_in / ORC_QK;
    long long nn = (long long)n_out;
#pragma omp parallel
    {
        float v[ORC_MAX_NB];
#pragma omp for schedule(static)
        for (long long n = 0; n < nn; n++) y[n] = gemv_row(w + (size_t)n * nb * ORC_BLOCK_BYTES, nb, x, v);
    }
    return 0;
}

int orc_gemm_q8_0(const uint8_t* w, size_t n_out, size_t k_in, const float* x, size_t m, float* y) {
    if (k_in == 0 || k_in % ORC_QK || n_out == 0 || m == 0) return 1;
    size_t nb = k_in / ORC_QK;
    /* activation rows -> Q8_0 (codes + f16 scales), same quantizer as weights */
    int8_t* xq = (int8_t*)malloc(m * k_in);
    float* xd = (float*)malloc(m * nb * sizeof(float));
    if (!xq || !xd) { free(xq); free(xd); return 2; }
    for (size_t r = 0; r < m; r++)
        for (size_t b = 0; b < nb; b++) {
            uint16_t d16;
            quantize_block(x + r * k_in + b * ORC_QK, &d16, xq + r * k_in + b * ORC_QK, NULL);
            xd[r * nb + b] = orc_f16_to_f32(d16);
        }
    long long total = (long long)(m * n_out);
#pragma omp parallel for schedule(static)
    for (long long t = 0; t < total; t++) {
        size_t r = (size_t)t / n_out, n = (size_t)t % n_out;
        const uint8_t* row = w + n * nb * ORC_BLOCK_BYTES;
        const int8_t* xr = xq + r * k_in;
        float acc = 0.0f;
        for (size_t g = 0; g < nb; g += ORC_GROUP_BLOCKS) {
            float a = 0.0f;
            size_t ge = g + ORC_GROUP_BLOCKS < nb ? g + ORC_GROUP_BLOCKS : nb;
            for (size_t b = g; b < ge; b++) {
                const uint8_t* blk = row + b * ORC_BLOCK_BYTES;
                const int8_t* q = (const int8_t*)(blk + 2);
                int32_t isum = 0;
                for (int j = 0; j < ORC_QK; j++) isum += (int32_t)q[j] * (int32_t)xr[b * ORC_QK + j];
                float s = blk_scale(blk) * xd[r * nb + b];
                if (g_seq_sums) acc = acc + (float)isum * s;
                else a = fmaf((float)isum, s, a);
            }
            if (!g_seq_sums) acc = acc + a;
        }
        y[r * n_out + n] = acc;
    }
    free(xq);
    free(xd);
    return 0;
}

/* 1 (default): more than one row goes through the W8A8 GEMM (activation
 * rows quantized to Q8_0).  0: every row goes through the W8A32 GEMV, which
 * the structure-pinning tests use so that an activation code landing on the
 * other side of a rounding midpoint cannot hide the rest of the decoder. */
static int g_act_quant = 1;
void orc_set_activation_quantization(int on) { g_act_quant = on ? 1 : 0; }

int orc_linear_forward(const uint8_t* w, size_t n_out, size_t k_in, const float* x, size_t m, float* y) {
    if (m == 1) return orc_gemv_q8_0(w, n_out, k_in, x, y);
    if (!g_act_quant) {
        for (size_t i = 0; i < m; i++) {
            int rc = orc_gemv_q8_0(w, n_out, k_in, x + i * k_in, y + i * n_out);
            if (rc) return rc;
        }
        return 0;
    }
    return orc_gemm_q8_0(w, n_out, k_in, x, m, y);
}

/* ------------------------------------------------------------------------ */
/* support ops                                                              */
/* ------------------------------------------------------------------------ */

/* src/rms_norm.rs:143-176: input rounded to bf16, sum of squares, mean,
 * inv = 1/sqrt(mean + eps), out = bf16((x*inv)*w). */
static void rms_norm_row(const float* x, const float* w, size_t dim, float eps, float* y, float* scratch) {
    for (size_t i = 0; i < dim; i++) {
        float v = site_bf16(x[i]);
        scratch[i] = v * v;
    }
    float ss = sum64(scratch, dim);
    float mean = ss / (float)dim;
    float inv = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < dim; i++) {
        float v = site_bf16(x[i]);
        y[i] = site_bf16((v * inv) * site_bf16(w[i]));
    }
}

int orc_rms_norm(const float* x, const float* weight, size_t rows, size_t dim, float eps, float* y) {
    if (dim == 0) return 1;
    float* scratch = (float*)malloc(dim * sizeof(float));
    if (!scratch) return 2;
    for (size_t r = 0; r < rows; r++) rms_norm_row(x + r * dim, weight, dim, eps, y + r * dim, scratch);
    free(scratch);
    return 0;
}

/* src/rope.rs:77-128: inv_freq[i] = 1/theta^(2i/rope_dim) (f64), each
 * frequency stored twice, cos/sin evaluated in f64 and cast to f32.
 * Tables are [max_pos][head_dim/2]. */
int orc_rope_tables(size_t head_dim, size_t max_pos, double theta, float* cos_t, float* sin_t) {
    if (head_dim % 4) return 1;
    size_t rope_dim = head_dim / 2, half = rope_dim / 2;
    double* inv_freq = (double*)malloc(half * sizeof(double));
    if (!inv_freq) return 2;
    for (size_t i = 0; i < half; i++) inv_freq[i] = 1.0 / pow(theta, (double)(2 * i) / (double)rope_dim);
    for (size_t p = 0; p < max_pos; p++)
        for (size_t i = 0; i < half; i++) {
            double f = (double)p * inv_freq[i];
            float c = (float)cos(f), s = (float)sin(f);
            cos_t[p * rope_dim + 2 * i] = c;
            cos_t[p * rope_dim + 2 * i + 1] = c;
            sin_t[p * rope_dim + 2 * i] = s;
            sin_t[p * rope_dim + 2 * i + 1] = s;
        }
    free(inv_freq);
    return 0;
}

/* src/rope.rs:270-297: out[d] = x[d]*c - x[d+R]*s, out[d+R] = x[d+R]*c + x[d]*s
 * with R = head_dim/2 and c, s taken at column 2*(d/2) of the table.
 * x is [heads][seq][head_dim]; positions are offset + l. */
int orc_rope_apply(const float* x, size_t heads, size_t seq, size_t head_dim, const float* cos_t,
                   const float* sin_t, size_t offset, float* y) {
    size_t R = head_dim / 2;
    for (size_t h = 0; h < heads; h++)
        for (size_t l = 0; l < seq; l++) {
            const float* xr = x + (h * seq + l) * head_dim;
            float* yr = y + (h * seq + l) * head_dim;
            const float* c = cos_t + (offset + l) * R;
            const float* s = sin_t + (offset + l) * R;
            for (size_t d = 0; d < R; d++) {
                float cv = c[d & ~(size_t)1], sv = s[d & ~(size_t)1];
                float x1 = xr[d], x2 = xr[d + R];
                yr[d] = x1 * cv - x2 * sv;
                yr[d + R] = x2 * cv + x1 * sv;
            }
        }
    return 0;
}

/* exp of the decoder's softmax and SiLU (orc_set_libm_exp) */
static float dec_exp(float x) { return g_libm_exp ? expf(x) : orc_expf(x); }

/* src/tensor.rs:1967-1978 (f32 branch). */
float orc_silu(float x) { return x / (1.0f + dec_exp(-x)); }

/* Iterator::max_by keeps the last of equal maxima (src/tensor.rs:2475-2480). */
uint32_t orc_argmax_last(const float* x, size_t n) {
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (!(x[i] < x[best])) best = i;
    return (uint32_t)best;
}

/* ------------------------------------------------------------------------ */
/* Qwen3 model (src/model.rs, src/transformer.rs, src/attention.rs, src/mlp.rs) */
/* ------------------------------------------------------------------------ */

typedef struct {
    const float *in_norm, *post_norm, *q_norm, *k_norm;
    const uint8_t *q, *k, *v, *o, *gate, *up, *down;
} orc_layer;

struct orc_model {
    orc_qwen3_config c;
    const uint8_t* embed;
    const float* final_norm;
    orc_layer* layers;
    float *cos_t, *sin_t;
    float *kc, *vc; /* [layer][kv_head][max_pos][head_dim] */
    size_t kv_len;
};

orc_model* orc_model_new(const orc_qwen3_config* cfg, const void* const* t) {
    orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
    if (!m) return NULL;
    m->c = *cfg;
    m->embed = (const uint8_t*)t[0];
    m->final_norm = (const float*)t[1];
    m->layers = (orc_layer*)calloc(cfg->num_layers, sizeof(orc_layer));
    size_t hd = cfg->head_dim, R = hd / 2;
    m->cos_t = (float*)malloc((size_t)cfg->max_positions * R * sizeof(float));
    m->sin_t = (float*)malloc((size_t)cfg->max_positions * R * sizeof(float));
    size_t kvsz = (size_t)cfg->num_layers * cfg->num_kv_heads * cfg->max_positions * hd;
    m->kc = (float*)calloc(kvsz, sizeof(float));
    m->vc = (float*)calloc(kvsz, sizeof(float));
    if (!m->layers || !m->cos_t || !m->sin_t || !m->kc || !m->vc) { orc_model_free(m); return NULL; }
    for (uint32_t l = 0; l < cfg->num_layers; l++) {
        const void* const* b = t + 2 + 11 * (size_t)l;
        orc_layer* L = &m->layers[l];
        L->in_norm = (const float*)b[0]; L->post_norm = (const float*)b[1];
        L->q_norm = (const float*)b[2]; L->k_norm = (const float*)b[3];
        L->q = (const uint8_t*)b[4]; L->k = (const uint8_t*)b[5]; L->v = (const uint8_t*)b[6];
        L->o = (const uint8_t*)b[7]; L->gate = (const uint8_t*)b[8]; L->up = (const uint8_t*)b[9];
        L->down = (const uint8_t*)b[10];
    }
    orc_rope_tables(hd, cfg->max_positions, cfg->rope_theta, m->cos_t, m->sin_t);
    return m;
}

void orc_model_free(orc_model* m) {
    if (!m) return;
    free(m->layers); free(m->cos_t); free(m->sin_t); free(m->kc); free(m->vc);
    free(m);
}

void orc_model_clear_kv_cache(orc_model* m) { m->kv_len = 0; }

/* One q-head attention row: q [hd], visible positions 0..L-1 of kv head kvh.
 * src/attention.rs:374-394 computes scores = q.k (sequential over d), times
 * 1/sqrt(hd), softmax (max, exp(x - max), sum, divide), then p.v.  Here the
 * positions are taken in segments of 64 (flash-decoding order, the same
 * arithmetic on every device):
 *   per segment c: s_j = (q.k_j sequential over d) * scale; m_c = max s_j;
 *     e_j = exp(s_j - m_c); l_c = SUM64(e); o_c[d] = sum_j e_j * v_j[d] (j in order);
 *   running (m, num[d], den) from (-inf, 0, 0): m' = max(m, m_c);
 *     a = exp(m - m'), b = exp(m_c - m'); num = num * a + b * o_c;
 *     den = den * a + b * l_c; m = m'.
 *   out[d] = num[d] / den.
 * With the plain sequential sums switch on, the reference's order is used. */
#define ORC_ATT_SEG 64
static void attend_kv(const float* K, const float* V, size_t hd, const float* q, size_t L, float* out, float* sc) {
    float scale = 1.0f / sqrtf((float)hd);
    if (g_seq_sums) {
        float mx = -INFINITY;
        for (size_t j = 0; j < L; j++) {
            float s = 0.0f;
            for (size_t d = 0; d < hd; d++) s = s + q[d] * K[j * hd + d];
            s = s * scale;
            sc[j] = s;
            if (s > mx) mx = s;
        }
        float sum = 0.0f;
        for (size_t j = 0; j < L; j++) { sc[j] = dec_exp(sc[j] - mx); sum = sum + sc[j]; }
        for (size_t j = 0; j < L; j++) sc[j] = sc[j] / sum;
        for (size_t d = 0; d < hd; d++) {
            float o = 0.0f;
            for (size_t j = 0; j < L; j++) o = o + sc[j] * V[j * hd + d];
            out[d] = o;
        }
        return;
    }
    float run_m = -INFINITY, den = 0.0f;
    for (size_t d = 0; d < hd; d++) out[d] = 0.0f; /* num */
    for (size_t js = 0; js < L; js += ORC_ATT_SEG) {
        size_t nj = L - js < ORC_ATT_SEG ? L - js : ORC_ATT_SEG;
        float mc = -INFINITY;
        for (size_t j = 0; j < nj; j++) {
            float s = 0.0f;
            const float* kr = K + (js + j) * hd;
            for (size_t d = 0; d < hd; d++) s = s + q[d] * kr[d];
            s = s * scale;
            sc[j] = s;
            if (s > mc) mc = s;
        }
        for (size_t j = 0; j < nj; j++) sc[j] = dec_exp(sc[j] - mc);
        float lc = sum64(sc, nj);
        float mn = run_m > mc ? run_m : mc;
        float a = dec_exp(run_m - mn), b = dec_exp(mc - mn);
        for (size_t d = 0; d < hd; d++) {
            float o = 0.0f;
            for (size_t j = 0; j < nj; j++) o = o + sc[j] * V[(js + j) * hd + d];
            out[d] = out[d] * a + b * o;
        }
        den = den * a + b * lc;
        run_m = mn;
    }
    for (size_t d = 0; d < hd; d++) out[d] = out[d] / den;
}

static void attend(const orc_model* m, size_t layer, size_t kvh, const float* q, size_t L, float* out, float* sc) {
    const orc_qwen3_config* c = &m->c;
    size_t hd = c->head_dim, P = c->max_positions;
    attend_kv(m->kc + ((layer * c->num_kv_heads + kvh) * P) * hd, m->vc + ((layer * c->num_kv_heads + kvh) * P) * hd,
              hd, q, L, out, sc);
}

static int model_forward(orc_model* m, const uint32_t* ids, size_t n, size_t offset, float* logits, float* hidden,
                         float* final_norm);

int orc_model_forward(orc_model* m, const uint32_t* ids, size_t n, size_t offset, float* logits) {
    return model_forward(m, ids, n, offset, logits, NULL, NULL);
}

/* Qwen3Model::forward_with_intermediates (src/model.rs:201-231): hidden is
 * [num_layers + 1][n][hidden] (embedding output, then each layer's output),
 * final_norm is [n][hidden]. */
int orc_model_forward_with_intermediates(orc_model* m, const uint32_t* ids, size_t n, size_t offset, float* hidden,
                                         float* final_norm, float* logits) {
    return model_forward(m, ids, n, offset, logits, hidden, final_norm);
}

static int model_forward(orc_model* m, const uint32_t* ids, size_t n, size_t offset, float* logits, float* hidden,
                         float* final_norm) {
    const orc_qwen3_config* c = &m->c;
    if (n == 0) return 1;
    if (offset != m->kv_len || offset + n > c->max_positions) return 3;
    size_t Hd = c->hidden_size, I = c->intermediate_size, hd = c->head_dim;
    size_t NH = c->num_heads, NKV = c->num_kv_heads, P = c->max_positions;
    size_t QD = NH * hd, KD = NKV * hd, R = hd / 2, groups = NH / NKV;
    size_t nbh = Hd / ORC_QK;
    for (size_t i = 0; i < n; i++)
        if (ids[i] >= c->vocab_size) return 3;

    float* H = (float*)malloc(n * Hd * sizeof(float));
    float* X = (float*)malloc(n * (Hd > QD ? Hd : QD) * sizeof(float));
    float* Q = (float*)malloc(n * QD * sizeof(float));
    float* K = (float*)malloc(n * KD * sizeof(float));
    float* Vv = (float*)malloc(n * KD * sizeof(float));
    float* A = (float*)malloc(n * QD * sizeof(float));
    float* O = (float*)malloc(n * Hd * sizeof(float));
    float* G = (float*)malloc(n * I * sizeof(float));
    float* U = (float*)malloc(n * I * sizeof(float));
    float* scratch = (float*)malloc((P > Hd ? P : Hd) * sizeof(float) * 2);
    float* tmp = (float*)malloc(hd * sizeof(float));
    if (!H || !X || !Q || !K || !Vv || !A || !O || !G || !U || !scratch || !tmp) {
        free(H); free(X); free(Q); free(K); free(Vv); free(A); free(O); free(G); free(U); free(scratch); free(tmp);
        return 2;
    }
    /* Embedding::forward (src/embedding.rs:137-152): row gather; rows are
     * dequantized Q8_0, exact in f32. */
    for (size_t i = 0; i < n; i++)
        orc_dequantize_q8_0(m->embed + (size_t)ids[i] * nbh * ORC_BLOCK_BYTES, Hd, H + i * Hd);
    if (hidden) memcpy(hidden, H, n * Hd * sizeof(float));

    for (size_t l = 0; l < c->num_layers; l++) {
        const orc_layer* L = &m->layers[l];
        orc_rms_norm(H, L->in_norm, n, Hd, c->rms_norm_eps, X);
        orc_linear_forward(L->q, QD, Hd, X, n, Q);
        orc_linear_forward(L->k, KD, Hd, X, n, K);
        orc_linear_forward(L->v, KD, Hd, X, n, Vv);
        /* per-head q/k RmsNorm then RoPE (src/attention.rs:350-364) */
        for (size_t i = 0; i < n; i++) {
            size_t pos = offset + i;
            const float* cs = m->cos_t + pos * R;
            const float* sn = m->sin_t + pos * R;
            for (size_t h = 0; h < NH + NKV; h++) {
                int isq = h < NH;
                float* src = isq ? Q + i * QD + h * hd : K + i * KD + (h - NH) * hd;
                rms_norm_row(src, isq ? L->q_norm : L->k_norm, hd, c->rms_norm_eps, tmp, scratch);
                float* dst;
                if (isq) dst = src;
                else dst = m->kc + ((l * NKV + (h - NH)) * P + pos) * hd;
                for (size_t d = 0; d < R; d++) {
                    float cv = cs[d & ~(size_t)1], sv = sn[d & ~(size_t)1];
                    float x1 = tmp[d], x2 = tmp[d + R];
                    dst[d] = x1 * cv - x2 * sv;
                    dst[d + R] = x2 * cv + x1 * sv;
                }
            }
            for (size_t h = 0; h < NKV; h++)
                memcpy(m->vc + ((l * NKV + h) * P + pos) * hd, Vv + i * KD + h * hd, hd * sizeof(float));
        }
        long long work = (long long)(n * NH);
#pragma omp parallel
        {
            float* sc = (float*)malloc((offset + n) * sizeof(float));
#pragma omp for schedule(static)
            for (long long t = 0; t < work; t++) {
                size_t i = (size_t)t / NH, h = (size_t)t % NH;
                attend(m, l, h / groups, Q + i * QD + h * hd, offset + i + 1, A + i * QD + h * hd, sc);
            }
            free(sc);
        }
        orc_linear_forward(L->o, Hd, QD, A, n, O);
        for (size_t t = 0; t < n * Hd; t++) H[t] = H[t] + O[t];
        orc_rms_norm(H, L->post_norm, n, Hd, c->rms_norm_eps, X);
        orc_linear_forward(L->gate, I, Hd, X, n, G);
        orc_linear_forward(L->up, I, Hd, X, n, U);
        for (size_t t = 0; t < n * I; t++) G[t] = orc_silu(G[t]) * U[t];
        orc_linear_forward(L->down, Hd, I, G, n, O);
        for (size_t t = 0; t < n * Hd; t++) H[t] = H[t] + O[t];
        if (hidden) memcpy(hidden + (l + 1) * n * Hd, H, n * Hd * sizeof(float));
    }
    if (final_norm) orc_rms_norm(H, m->final_norm, n, Hd, c->rms_norm_eps, final_norm);
    m->kv_len = offset + n;
    /* final norm of the last position, then lm_head GEMV (src/model.rs:357-371) */
    orc_rms_norm(H + (n - 1) * Hd, m->final_norm, 1, Hd, c->rms_norm_eps, X);
    orc_gemv_q8_0(m->embed, c->vocab_size, Hd, X, logits);
    free(H); free(X); free(Q); free(K); free(Vv); free(A); free(O); free(G); free(U); free(scratch); free(tmp);
    return 0;
}

/* src/generate.rs:611-664 with the greedy sampler; no EOS stop.
 * feed_first = 0: each decode step forwards the token generated last (the
 * loop the library implements).  feed_first = 1: the loop as the reference
 * writes it -- the `let next_token` inside the loop body (generate.rs:650)
 * shadows the outer binding (generate.rs:632) only for the rest of that
 * iteration, so every decode step forwards the FIRST generated token
 * (generate.rs:647) at offset prefill_len + generated - 1. */
int orc_generate_greedy_ex(orc_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new, int feed_first,
                           uint32_t* out_tokens, float* out_margins) {
    if (n_prompt == 0 || max_new == 0) return 1;
    float* logits = (float*)malloc((size_t)m->c.vocab_size * sizeof(float));
    if (!logits) return 2;
    orc_model_clear_kv_cache(m);
    int rc = 0;
    uint32_t tok = 0;
    for (size_t t = 0; t < max_new; t++) {
        if (t == 0) rc = orc_model_forward(m, prompt, n_prompt, 0, logits);
        else rc = orc_model_forward(m, feed_first ? &out_tokens[0] : &tok, 1, n_prompt + t - 1, logits);
        if (rc) break;
        tok = orc_argmax_last(logits, m->c.vocab_size);
        out_tokens[t] = tok;
        if (out_margins) {
            float best = logits[tok], second = -INFINITY;
            for (size_t i = 0; i < m->c.vocab_size; i++)
                if (i != tok && logits[i] > second) second = logits[i];
            out_margins[t] = best - second;
        }
    }
    free(logits);
    return rc;
}

int orc_generate_greedy(orc_model* m, const uint32_t* prompt, size_t n_prompt, size_t max_new,
                        uint32_t* out_tokens, float* out_margins) {
    return orc_generate_greedy_ex(m, prompt, n_prompt, max_new, 0, out_tokens, out_margins);
}

/* ------------------------------------------------------------------------ */
/* Qwen3-MoE decoder layer, decode step of T independent sequences           */
/* ------------------------------------------------------------------------ */
/* No MoE code exists in the reference; the layer is the Qwen3-MoE block
 * (Qwen3-30B-A3B style) assembled from the reference's decoder numerics above
 * (src/transformer.rs:180-204 residual structure, src/attention.rs:318-403
 * attention, src/mlp.rs:151-164 SwiGLU) with these choices, which the GPU
 * path follows bit for bit:
 *   - every projection is applied per token (M = 1, the W8A32 GEMV order), so
 *     a token's result does not depend on the other tokens of the batch;
 *   - router: m = max s, e_i = exp(s_i - m), S = SUM64(e), p_i = e_i / S;
 *     top-k by p, descending, ties to the lower expert index; the k weights
 *     are renormalised: w_r = p_r / (((p_0 + p_1) + p_2) + ...) in rank order;
 *   - expert e: y_e = down(silu(gate x) * up x), x = post-attention RmsNorm;
 *   - combine in ascending expert index: acc = 0; acc = acc + w_e * y_e;
 *     out = h2 + acc (h2 = input + attention output). */

struct orc_moe {
    orc_moe_config c;
    const void* const* t; /* per layer: 8 + 3E pointers */
    float *cos_t, *sin_t;
    float *kc, *vc; /* [layer][seq][kv_head][max_pos][head_dim] */
};

orc_moe* orc_moe_new(const orc_moe_config* cfg, const void* const* tensors) {
    orc_moe* m = (orc_moe*)calloc(1, sizeof(orc_moe));
    if (!m) return NULL;
    m->c = *cfg;
    m->t = tensors;
    size_t hd = cfg->head_dim, R = hd / 2;
    m->cos_t = (float*)malloc((size_t)cfg->max_positions * R * sizeof(float));
    m->sin_t = (float*)malloc((size_t)cfg->max_positions * R * sizeof(float));
    size_t kvsz = (size_t)cfg->num_layers * cfg->max_batch * cfg->num_kv_heads * cfg->max_positions * hd;
    m->kc = (float*)calloc(kvsz, sizeof(float));
    m->vc = (float*)calloc(kvsz, sizeof(float));
    if (!m->cos_t || !m->sin_t || !m->kc || !m->vc) { orc_moe_free(m); return NULL; }
    orc_rope_tables(hd, cfg->max_positions, cfg->rope_theta, m->cos_t, m->sin_t);
    return m;
}

void orc_moe_free(orc_moe* m) {
    if (!m) return;
    free(m->cos_t); free(m->sin_t); free(m->kc); free(m->vc);
    free(m);
}

int orc_moe_route(const float* scores, size_t T, size_t E, size_t k, uint32_t* ids, float* weights) {
    if (E == 0 || k == 0 || k > E) return 1;
    float* e = (float*)malloc(E * sizeof(float));
    unsigned char* used = (unsigned char*)malloc(E);
    if (!e || !used) { free(e); free(used); return 2; }
    for (size_t t = 0; t < T; t++) {
        const float* s = scores + t * E;
        float mx = -INFINITY;
        for (size_t i = 0; i < E; i++) if (s[i] > mx) mx = s[i];
        for (size_t i = 0; i < E; i++) e[i] = orc_expf(s[i] - mx);
        float S = sum64(e, E);
        for (size_t i = 0; i < E; i++) { e[i] = e[i] / S; used[i] = 0; }
        float tot = 0.0f;
        for (size_t r = 0; r < k; r++) {
            size_t best = E;
            for (size_t i = 0; i < E; i++)
                if (!used[i] && (best == E || e[i] > e[best])) best = i;
            used[best] = 1;
            ids[t * k + r] = (uint32_t)best;
            weights[t * k + r] = e[best];
            tot = tot + e[best];
        }
        for (size_t r = 0; r < k; r++) weights[t * k + r] = weights[t * k + r] / tot;
    }
    free(e); free(used);
    return 0;
}

/* One decode step of T sequences (sequence t in KV slot t at pos[t]).  The
 * attention projections of all T tokens are one Linear::forward each
 * (orc_linear_forward: the GEMV at T = 1, the W8A8 GEMM at T > 1, as the
 * reference's Linear::forward over an [T, hidden] input), so a token's
 * result depends on whether it runs alone or in a batch, never on the other
 * tokens of the batch; the experts run per token (single-vector GEMVs). */
int orc_moe_forward(orc_moe* m, float* hidden, const float* scores, const uint32_t* pos, size_t T) {
    const orc_moe_config* c = &m->c;
    size_t H = c->hidden_size, hd = c->head_dim, NH = c->num_heads, NKV = c->num_kv_heads;
    size_t E = c->num_experts, K = c->top_k, I = c->expert_intermediate_size, P = c->max_positions;
    size_t QD = NH * hd, KD = NKV * hd, R = hd / 2, groups = NH / NKV;
    if (T == 0 || T > c->max_batch) return 1;
    for (size_t t = 0; t < T; t++) if (pos[t] >= P) return 3;
    float* X = (float*)malloc(T * H * sizeof(float));
    float* Q = (float*)malloc(T * QD * sizeof(float));
    float* Kx = (float*)malloc(T * KD * sizeof(float));
    float* Vx = (float*)malloc(T * KD * sizeof(float));
    float* A = (float*)malloc(T * QD * sizeof(float));
    float* O = (float*)malloc(T * H * sizeof(float));
    float* G = (float*)malloc(I * sizeof(float));
    float* U = (float*)malloc(I * sizeof(float));
    float* Y = (float*)malloc(H * sizeof(float));
    float* acc = (float*)malloc(H * sizeof(float));
    float* sc = (float*)malloc((P > H ? P : H) * 2 * sizeof(float));
    float* tmp = (float*)malloc(hd * sizeof(float));
    uint32_t* ids = (uint32_t*)malloc(T * K * sizeof(uint32_t));
    float* wts = (float*)malloc(T * K * sizeof(float));
    int rc = 0;
    if (!X || !Q || !Kx || !Vx || !A || !O || !G || !U || !Y || !acc || !sc || !tmp || !ids || !wts) { rc = 2; goto done; }
    for (size_t l = 0; l < c->num_layers; l++) {
        const void* const* b = m->t + (8 + 3 * E) * l;
        const float *in_norm = (const float*)b[0], *post_norm = (const float*)b[1];
        const float *q_norm = (const float*)b[2], *k_norm = (const float*)b[3];
        orc_moe_route(scores + l * T * E, T, E, K, ids, wts);
        orc_rms_norm(hidden, in_norm, T, H, c->rms_norm_eps, X);
        if ((rc = orc_linear_forward((const uint8_t*)b[4], QD, H, X, T, Q)) ||
            (rc = orc_linear_forward((const uint8_t*)b[5], KD, H, X, T, Kx)) ||
            (rc = orc_linear_forward((const uint8_t*)b[6], KD, H, X, T, Vx)))
            goto done;
        for (size_t t = 0; t < T; t++) {
            size_t p = pos[t];
            float* kc = m->kc + ((l * c->max_batch + t) * NKV) * P * hd;
            float* vc = m->vc + ((l * c->max_batch + t) * NKV) * P * hd;
            float *Qt = Q + t * QD, *Kt = Kx + t * KD, *Vt = Vx + t * KD;
            const float* cs = m->cos_t + p * R;
            const float* sn = m->sin_t + p * R;
            for (size_t hh = 0; hh < NH + NKV; hh++) {
                int isq = hh < NH;
                float* src = isq ? Qt + hh * hd : Kt + (hh - NH) * hd;
                rms_norm_row(src, isq ? q_norm : k_norm, hd, c->rms_norm_eps, tmp, sc);
                float* dst = isq ? src : kc + ((hh - NH) * P + p) * hd;
                for (size_t d = 0; d < R; d++) {
                    float cv = cs[d & ~(size_t)1], sv = sn[d & ~(size_t)1];
                    float x1 = tmp[d], x2 = tmp[d + R];
                    dst[d] = x1 * cv - x2 * sv;
                    dst[d + R] = x2 * cv + x1 * sv;
                }
            }
            for (size_t hh = 0; hh < NKV; hh++) memcpy(vc + (hh * P + p) * hd, Vt + hh * hd, hd * sizeof(float));
            for (size_t hh = 0; hh < NH; hh++) {
                size_t kvh = hh / groups;
                attend_kv(kc + kvh * P * hd, vc + kvh * P * hd, hd, Qt + hh * hd, p + 1, A + t * QD + hh * hd, sc);
            }
        }
        if ((rc = orc_linear_forward((const uint8_t*)b[7], H, QD, A, T, O))) goto done;
        for (size_t i = 0; i < T * H; i++) hidden[i] = hidden[i] + O[i];   /* h2 */
        for (size_t t = 0; t < T; t++) {
            float* h = hidden + t * H;
            orc_rms_norm(h, post_norm, 1, H, c->rms_norm_eps, X);
            for (size_t i = 0; i < H; i++) acc[i] = 0.0f;
            for (size_t e = 0; e < E; e++) {
                float w = 0.0f;
                int hit = 0;
                for (size_t r = 0; r < K; r++) if (ids[t * K + r] == e) { w = wts[t * K + r]; hit = 1; }
                if (!hit) continue;
                orc_gemv_q8_0((const uint8_t*)b[8 + e], I, H, X, G);
                orc_gemv_q8_0((const uint8_t*)b[8 + E + e], I, H, X, U);
                for (size_t i = 0; i < I; i++) G[i] = orc_silu(G[i]) * U[i];
                orc_gemv_q8_0((const uint8_t*)b[8 + 2 * E + e], H, I, G, Y);
                for (size_t i = 0; i < H; i++) acc[i] = acc[i] + w * Y[i];
            }
            for (size_t i = 0; i < H; i++) h[i] = h[i] + acc[i];
        }
    }
done:
    free(X); free(Q); free(Kx); free(Vx); free(A); free(O); free(G); free(U); free(Y); free(acc); free(sc); free(tmp);
    free(ids); free(wts);
    return rc;
}

/* ---- sampling (the library's rule; the reference's samplers are argmax
 * stubs, src/generate.rs:191-329) ------------------------------------------
 * penalty per earlier occurrence (src/generate.rs:353-380), T = 0 greedy
 * (last index on ties), else z = x / T, order by z descending (lower index
 * first on ties), top_k, integer weights w = floor(2^32 * exp(z - z0)) (0 for
 * NaN), prefix sums C exact in 64 bits, nucleus end = first C >= thr with
 * thr = ceil(S * floor(top_p * 2^24) / 2^24), u24 = SplitMix64(seed + step *
 * golden) >> 40, r = floor(C_end * u24 / 2^24), token = first C > r (the
 * first entry when C_end = 0).  Sorting: qsort of distinct 64-bit keys
 * (value bits above the index or its complement), sums sequential. */
static uint32_t orc_order_bits(float z) {
    uint32_t b;
    memcpy(&b, &z, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
static float orc_from_order(uint32_t k) {
    uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    float f;
    memcpy(&f, &b, 4);
    return f;
}
static int orc_cmp_desc_u64(const void* a, const void* b) {
    const uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return x < y ? 1 : (x > y ? -1 : 0);
}
static uint64_t orc_splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static uint64_t orc_weight(float z, float z0) {
    const float e = orc_expf(z - z0);
    if (!(e > 0.0f)) return 0;
    return (uint64_t)fminf(e * 4294967296.0f, 4294967296.0f);
}

int64_t orc_sample(const float* logits, size_t V, const uint32_t* counts, float T, uint32_t top_k, float top_p,
                   float penalty, uint64_t seed, uint32_t step) {
    if (V == 0) return -1;
    uint64_t* keys = (uint64_t*)malloc(V * sizeof(uint64_t));
    if (!keys) return -1;
    for (size_t i = 0; i < V; i++) {
        float x = logits[i];
        if (fabsf(penalty - 1.0f) >= 1e-6f && counts)
            for (uint32_t c = 0; c < counts[i]; c++) {
                if (x > 0.0f) x = x / penalty;
                else if (x < 0.0f) x = x * penalty;
            }
        const float z = T > 0.0f ? x / T : x;
        const uint32_t lo = T > 0.0f ? ~(uint32_t)i : (uint32_t)i;
        keys[i] = ((uint64_t)orc_order_bits(z) << 32) | lo;
    }
    qsort(keys, V, sizeof(uint64_t), orc_cmp_desc_u64);
    if (!(T > 0.0f)) {
        const int64_t token = (uint32_t)keys[0];
        free(keys);
        return token;
    }
    const size_t K = top_k > 0 && top_k < V ? top_k : V;
    const float z0 = orc_from_order((uint32_t)(keys[0] >> 32));
    uint64_t* C = (uint64_t*)malloc(K * sizeof(uint64_t));
    if (!C) {
        free(keys);
        return -1;
    }
    uint64_t acc = 0;
    for (size_t j = 0; j < K; j++) {
        acc += orc_weight(orc_from_order((uint32_t)(keys[j] >> 32)), z0);
        C[j] = acc;
    }
    const uint64_t S = C[K - 1];
    uint64_t c_end = S;
    if (top_p < 1.0f) {
        const uint64_t p24 = (uint64_t)(top_p * 16777216.0f);
        const unsigned __int128 prod = (unsigned __int128)S * p24;
        const uint64_t thr = (uint64_t)(prod >> 24) + ((prod & 0xFFFFFFu) ? 1u : 0u);
        for (size_t j = 0; j < K; j++)
            if (C[j] >= thr) {
                c_end = C[j];
                break;
            }
    }
    const uint64_t u24 = orc_splitmix64(seed + (uint64_t)step * 0x9E3779B97F4A7C15ull) >> 40;
    const uint64_t r = (uint64_t)(((unsigned __int128)c_end * u24) >> 24);
    size_t pick = 0;
    if (c_end > 0)
        for (size_t j = 0; j < K; j++)
            if (C[j] > r) {
                pick = j;
                break;
            }
    const int64_t token = ~(uint32_t)keys[pick];
    free(C);
    free(keys);
    return token;
}
