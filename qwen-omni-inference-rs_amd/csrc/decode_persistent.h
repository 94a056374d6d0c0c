// decode_persistent.h -- host interface of the persistent greedy decode
// kernel (decode_persistent.hip).
#pragma once

#include "lq8_internal.h"

namespace lq8 {

constexpr int PERSIST_THREADS = 512;
constexpr int PERSIST_FETCH = 16;  // hand-off words one thread fetches per phase, at most
constexpr int PERSIST_NCH = 8;     // o-projection input chunks (partial sums per output row), at most

// Device pointers of one decoder layer.
struct PLayer {
    const int8_t *qkv_c, *o_c, *gu_c, *dn_c;
    const uint16_t *qkv_s, *o_s, *gu_s, *dn_s;
    const float *in_norm, *post_norm, *q_norm, *k_norm;
};

struct PersistShape {
    int H, I, NH, NKV, head_dim, max_pos;
};

// Work split and LDS map of one shape on P workgroups (persist_layout).
struct PersistLayout {
    int hc;             // block pairs per wave group of a hidden-long tile (2: hidden <= 1024, 4: <= 2048)
    int csO, nchO;      // o projection: input chunks of csO blocks (a power of two), nchO of them
    int csD, nchD;      // down projection: input chunks of csD block pairs (a power of two), nchD of them
    int cdir;           // steps with at most cdir segments: P3 combines the partials itself
    int fr, xs_off, gs_off, red_off, att_floats, comb_floats;  // LDS, in floats (combine: inside att_floats)
    int smem_bytes;
    size_t words;       // tagged hand-off words of all buffers
};

struct PersistArgs {
    const PLayer* layers;  // device [L]
    int L;
    const int8_t* emb_c;   // tied embedding / lm_head [vocab][H]
    const uint16_t* emb_s;
    const float* final_norm;
    const float* cos_t;    // [max_pos][64]
    const float* sin_t;
    float* kc;             // [L][NKV][max_pos][128]
    float* vc;
    int H, I, NH, NKV, max_pos, cmax, vocab;
    float eps, scale;
    int csO, nchO;
    int csD, nchD;
    int cdir;          // P3 combines the segment partials itself while C <= cdir
    // tagged hand-off words (f32 bits | tag << 32)
    uint64_t* qkvb;   // [L][QKV]: q|k|v projection
    uint64_t* partb;  // [L][cmax][NH][ATT_PART_STRIDE]: attention partials per (segment, head)
    uint64_t* attb;   // [L][NH * 128]: attention output (the segments combined), heads concatenated
    uint64_t* resb;   // [L + 1][(1 + nchO) * H]: layer input h, then the o projection's chunk sums [nchO][H]
    uint64_t* h2b;    // [L][(1 + nchD) * H]: h + o projection (the MLP's input and residual), then the down
                      // projection's chunk sums [nchD][H]
    uint64_t* actb;   // [L][I]: silu(gate) * up
    uint64_t* argb;   // [2][P][2]: each workgroup's greedy pick (value, index bits), by the step tag's parity
    unsigned* abort_flag;
    // steps: positions pos0 .. pos0 + steps - 1; tokens_out[step0 + s] gets step s's pick
    int pos0, steps, step0, feed_first;
    unsigned tag0;     // tag of step s: tag0 + s (never 0)
    uint32_t* d_tok;   // input token of the first step; the last pick on exit
    uint32_t* tokens_out;
    int* d_pos;
    int* d_step;
    // LDS map (floats) and size (bytes)
    int fr, xs_off, gs_off, red_off, smem_bytes;
};

// false when the shape does not fit the kernel's limits on P workgroups
bool persist_layout(const PersistShape& s, int P, PersistLayout* out);
bool persist_supported(const PersistShape& s, int num_cus);
// the kernel instance's block pairs per wave group of a hidden-long tile
int persist_pairs_per_wave(int hidden);
// d_args: the argument block in device memory (read by the kernel throughout)
// ch5: block pairs per wave group of the down items (csD / waves per workgroup)
// hc: persist_pairs_per_wave(hidden)
// long_ctx: the instance with the combining attention items, for steps whose
// positions have more than cdir segments (the other instance requires
// pos0 + steps <= cdir * ATT_SEG)
lq8_status launch_decode_persistent(hipStream_t st, const PersistArgs* d_args, int smem_bytes, int num_wg, int ch5,
                                    int hc, bool long_ctx);

}  // namespace lq8
