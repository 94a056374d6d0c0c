// gemv_device.h -- the Q8_0 GEMV's per-chunk arithmetic, shared by the GEMV
// kernels (gemv.hip) and the persistent decode kernel (decode_persistent.hip):
// the 16-code fmaf chain, the greedy pick step, and the staged-input
// transforms (bf16 rounding, RmsNorm output element, silu(gate) * up).
#pragma once

#include "lq8_internal.h"
#include "lq8_numerics.h"

namespace lq8 {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
// fmaf chain over the 16 codes in v against x[0..15], from +0.
__device__ __forceinline__ float dot16(u32x4 v, const float* __restrict__ x) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 xv = *(const float4*)(x + 4 * i);
        p = fmaf((float)(int8_t)(w[i] & 0xFF), xv.x, p);
        p = fmaf((float)(int8_t)((w[i] >> 8) & 0xFF), xv.y, p);
        p = fmaf((float)(int8_t)((w[i] >> 16) & 0xFF), xv.z, p);
        p = fmaf((float)(int8_t)(w[i] >> 24), xv.w, p);
    }
    return p;
}

// One level of the greedy pick between lane l and lane l ^ D: maximum, last
// index on ties.
template <int D>
__device__ __forceinline__ void argmax_step(float& bv, int& bi) {
    const float ov = lane_xor<D>(bv);
    const int oi = lane_xor_int<D>(bi);
    if (ov > bv || (ov == bv && oi > bi)) {
        bv = ov;
        bi = oi;
    }
}

__device__ __forceinline__ float4 bf16_round4(float4 v) {
    return make_float4(bf16_round(v.x), bf16_round(v.y), bf16_round(v.z), bf16_round(v.w));
}
__device__ __forceinline__ float silu_mul(float g, float u) { return __fdiv_rn(g, 1.0f + expf_cr(-g)) * u; }
// RmsNorm output element (src/rms_norm.rs:159-173): bf16((v * inv) * bf16(w)), v = bf16(x)
__device__ __forceinline__ float4 norm4(float4 v, float4 w, float inv) {
    return make_float4(bf16_round((v.x * inv) * bf16_round(w.x)), bf16_round((v.y * inv) * bf16_round(w.y)),
                       bf16_round((v.z * inv) * bf16_round(w.z)), bf16_round((v.w * inv) * bf16_round(w.w)));
}

}  // namespace lq8
