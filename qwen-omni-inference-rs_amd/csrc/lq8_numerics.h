// lq8_numerics.h -- device scalar numerics with fixed, documented rounding.
//
// The library is compiled with -ffp-contract=off; every fused multiply-add
// below is an explicit fmaf/fma, every division and square root is the
// correctly rounded one.  The same operation sequences, run on any IEEE
// machine, give the same bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace lq8 {

__device__ __forceinline__ float bf16_round(float x) {
    // src/bf16.rs:112-131: add 0x7FFF + lsb, keep the upper 16 bits.
    uint32_t b = __float_as_uint(x);
    uint32_t bias = 0x7FFFu + ((b >> 16) & 1u);
    return __uint_as_float(((b + bias) >> 16) << 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
    _Float16 h = (_Float16)x;  // v_cvt_f16_f32, round to nearest even
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);  // exact
}

// exp evaluated in double (Cody-Waite reduction, degree-13 Taylor), rounded
// once to float.  Every step is an IEEE operation.
__device__ __forceinline__ float expf_cr(float xf) {
    if (xf != xf) return xf;
    if (xf > 89.0f) return __builtin_huge_valf();
    if (xf < -110.0f) return 0.0f;
    double x = (double)xf;
    double k = rint(x * 1.4426950408889634074);
    double r = fma(-k, 6.93147180369123816490e-01, x);
    r = fma(-k, 1.90821492927058770002e-10, r);
    double p = 1.0 / 6227020800.0;
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

// Rust `f32 as i8`: saturating, NaN -> 0.
__device__ __forceinline__ int sat_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int)v;
}

// ---- cross-lane exchange without the LDS path (gfx950) ----------------------
// lane_xor<D>(v): the value v of lane l ^ D (exactly the __shfl_xor partner)
// from VALU lane moves: v_permlane32_swap / v_permlane16_swap (the same
// register as both operands returns, in every lane, the values of the lower
// and the upper lane of the pair), DPP row_ror:8 (lane i of a 16-lane row
// reads lane (i - 8) mod 16 = i ^ 8), row_shl:4 / row_shr:4 (lanes i + 4 and
// i - 4; the one inside the row is i ^ 4) and quad_perm (i ^ 2, i ^ 1).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

struct LanePair {
    float lo, hi;  // values of lanes l & ~D and l | D
};

__device__ __forceinline__ LanePair lanes32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return {__uint_as_float(p[0]), __uint_as_float(p[1])};
}

__device__ __forceinline__ LanePair lanes16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return {__uint_as_float(p[0]), __uint_as_float(p[1])};
}

// Two registers through one swap (rows are 16-lane groups, halves 32-lane
// groups; a == b gives lanes16 / lanes32):
//   rows16(a, b):   .lo = rows (a0, b0, a2, b2), .hi = rows (a1, b1, a3, b3)
//   halves32(a, b): .lo = halves (a0, b0),       .hi = halves (a1, b1)
// so .lo + .hi sums the row (half) pairs of both registers at once.
__device__ __forceinline__ LanePair rows16(float a, float b) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return {__uint_as_float(p[0]), __uint_as_float(p[1])};
}

__device__ __forceinline__ LanePair halves32(float a, float b) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return {__uint_as_float(p[0]), __uint_as_float(p[1])};
}

template <int D>
__device__ __forceinline__ float lane_xor(float v) {
    static_assert(D == 1 || D == 2 || D == 4 || D == 8 || D == 16 || D == 32, "xor distance");
    const int lane = __lane_id();
    if constexpr (D == 32) {
        const LanePair p = lanes32(v);
        return (lane & 32) ? p.lo : p.hi;
    } else if constexpr (D == 16) {
        const LanePair p = lanes16(v);
        return (lane & 16) ? p.lo : p.hi;
    } else if constexpr (D == 8) {
        return dpp_move<0x128>(v);  // row_ror:8
    } else if constexpr (D == 4) {
        const float up = dpp_move<0x104>(v), down = dpp_move<0x114>(v);  // row_shl:4, row_shr:4
        return (lane & 4) ? down : up;
    } else if constexpr (D == 2) {
        return dpp_move<0x4E>(v);  // quad_perm [2, 3, 0, 1]
    } else {
        return dpp_move<0xB1>(v);  // quad_perm [1, 0, 3, 2]
    }
}

template <int D>
__device__ __forceinline__ int lane_xor_int(int v) {
    return __builtin_bit_cast(int, lane_xor<D>(__builtin_bit_cast(float, v)));
}

// SUM64 fold of one 64-lane wave's partials: a = a + (lane l ^ d's a) for
// d = 32, 16, 8, 4, 2, 1.
__device__ __forceinline__ float wave_sum64(float a) {
    a = a + lane_xor<32>(a);
    a = a + lane_xor<16>(a);
    a = a + lane_xor<8>(a);
    a = a + lane_xor<4>(a);
    a = a + lane_xor<2>(a);
    a = a + lane_xor<1>(a);
    return a;
}

// Q8_0 block quantizer (GGML quantize_row_q8_0 / candle BlockQ8_0::from_float):
// amax ignores NaN, d = amax/127, id = d ? 1/d : 0, q = round_half_away(x*id).
struct QBlock {
    float d;        // f32 scale used for the codes
    uint16_t d16;   // stored f16 scale
};

__device__ __forceinline__ float block_amax(const float* x) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        float v = fabsf(x[j]);
        if (v > amax) amax = v;
    }
    return amax;
}

__device__ __forceinline__ QBlock block_scale(float amax) {
    QBlock b;
    b.d = __fdiv_rn(amax, 127.0f);
    b.d16 = f32_to_f16_bits(b.d);
    return b;
}

__device__ __forceinline__ float block_inv(float d) { return d != 0.0f ? __fdiv_rn(1.0f, d) : 0.0f; }

__device__ __forceinline__ int quant_code(float x, float id) { return sat_i8(roundf(x * id)); }

}  // namespace lq8
