// decode_persistent.h -- host interface of the persistent greedy decode
// kernel (decode_persistent.hip).
#pragma once

#include "lq8_internal.h"

namespace lq8 {

constexpr int PERSIST_THREADS = 256;

// Device pointers of one decoder layer.
struct PLayer {
    const int8_t *qkv_c, *o_c, *gu_c, *dn_c;
    const uint16_t *qkv_s, *o_s, *gu_s, *dn_s;
    const float *in_norm, *post_norm, *q_norm, *k_norm;
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
    // tagged hand-off words (f32 bits | tag << 32), per layer
    uint64_t* qkvb;   // [L][QKV]
    uint64_t* partb;  // [L][cmax][NH][ATT_PART_STRIDE]
    uint64_t* attnb;  // [L][NH * 128]: the combined attention output
    uint64_t* h2b;    // [L][H]
    uint64_t* actb;   // [L][I]
    uint64_t* hb;     // [L][H]
    uint64_t* argb;   // [P][2]: each workgroup's greedy pick (value, index bits)
    unsigned* cntb;   // [L][NKV][16]: per kv head, the step's segment arrivals (back to 0 after the last)
    unsigned* abort_flag;
    // steps: positions pos0 .. pos0 + steps - 1; tokens_out[step0 + s] gets step s's pick
    int pos0, steps, step0, feed_first;
    unsigned tag0;     // tag of step s: tag0 + s (never 0)
    uint32_t* d_tok;   // input token of the first step; the last pick on exit
    uint32_t* tokens_out;
    int* d_pos;
    int* d_step;
    // LDS layout (floats) and size (bytes)
    int xs_floats, region_a, smem_bytes;
};

struct PersistShape {
    int H, I, NH, NKV, head_dim, max_pos;
};

bool persist_supported(const PersistShape& s, int num_cus);
size_t persist_xs_floats(const PersistShape& s);
size_t persist_region_a(const PersistShape& s);
size_t persist_smem_bytes(const PersistShape& s);
// d_args: the argument block in device memory (read by the kernel throughout)
lq8_status launch_decode_persistent(hipStream_t st, const PersistArgs* d_args, int smem_bytes, int num_wg);

}  // namespace lq8
