// Bit-exact glm_act activations and fp32_rsqrt as device functions.
//
// Restates tools/glm_model_q4k_ref.py:96-116 (fp32_rsqrt) and :214-299 (sigmoid core,
// glm_sigmoid, glm_silu).  Every fp32 op is one IEEE op (the library is built with
// -ffp-contract=off), and the integer steps act on the raw bit patterns, so the results
// match the reference bit for bit, including its FTZ and clamping corners.
#pragma once

#include "common.hpp"

namespace aipu {

// Magic-seed reciprocal square root with exactly two Newton steps.
// NaN, negative (incl. -0), zero and subnormal inputs -> quiet NaN; +inf -> +0.
__device__ __forceinline__ float glm_rsqrt(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t e = (u >> 23) & 0xFFu, man = u & 0x7FFFFFu;
    if ((e == 0xFFu && man != 0u) || (u >> 31) != 0u || e == 0u) return __uint_as_float(0x7FC00000u);
    if (e == 0xFFu) return 0.0f;
    const float xh = 0.5f * x;
    float y = __uint_as_float(0x5F3759DFu - (u >> 1));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float yy = y * y;
        const float xyy = xh * yy;
        const float t = 1.5f - xyy;
        y = y * t;
    }
    return y;
}

// fp32 -> int with the magnitude rounded half-up (arguments are bounded by |16*log2 e|).
__device__ __forceinline__ int act_round_half_up(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t e = (u >> 23) & 0xFFu;
    const uint32_t m = 0x800000u | (u & 0x7FFFFFu);
    int r;
    if (e < 127u) {
        r = (e == 126u) ? 1 : 0;
    } else {
        const int sh = 23 - ((int)e - 127);
        r = (int)((m >> sh) & 0xFFu) + (int)((m >> (sh - 1)) & 1u);
    }
    return (u >> 31) ? -r : r;
}

// inf/NaN -> signed 16.0
__device__ __forceinline__ float act_sanitize(float x) {
    const uint32_t u = __float_as_uint(x);
    if (((u >> 23) & 0xFFu) == 0xFFu) return __uint_as_float((u & 0x80000000u) | 0x41800000u);
    return x;
}

// Unrounded fp32 sigmoid core.
__device__ __forceinline__ float glm_sigmoid_f32(float x) {
    float xs = act_sanitize(x);
    uint32_t u = __float_as_uint(xs);
    if ((u & 0x7FFFFFFFu) >= 0x41800000u) xs = __uint_as_float((u & 0x80000000u) | 0x41800000u);
    const float z = __uint_as_float(__float_as_uint(xs) ^ 0x80000000u);
    const float kf = z * __uint_as_float(0x3FB8AA3Bu);            // z * log2(e)
    int k = act_round_half_up(kf);
    k = k > 64 ? 64 : (k < -64 ? -64 : k);
    const float kl = (float)k * __uint_as_float(0x3F317218u);     // k * ln 2
    const float r = z - kl;
    float p = __uint_as_float(0x3D2AAAABu) + r * __uint_as_float(0x3C088889u);
    p = __uint_as_float(0x3E2AAAABu) + r * p;
    p = __uint_as_float(0x3F000000u) + r * p;
    p = 1.0f + r * p;
    p = 1.0f + r * p;
    const uint32_t pu = __float_as_uint(p);
    const int en = (int)((pu >> 23) & 0xFFu) + k;
    const uint32_t sg = pu & 0x80000000u;
    uint32_t ex;
    if (en >= 255) ex = sg | (0xFEu << 23) | (pu & 0x7FFFFFu);
    else if (en <= 0) ex = sg;
    else ex = sg | ((uint32_t)en << 23) | (pu & 0x7FFFFFu);
    const float d = 1.0f + __uint_as_float(ex);
    const float t = glm_rsqrt(d);
    return t * t;
}

__device__ __forceinline__ uint32_t glm_sigmoid_bf16(uint32_t xb) {
    return bf16_rne(glm_sigmoid_f32(bf16_to_f32(xb)));
}

__device__ __forceinline__ uint32_t glm_silu_bf16(uint32_t xb) {
    const float x = bf16_to_f32(xb);
    const float s = glm_sigmoid_f32(x);
    return bf16_rne(s * act_sanitize(x));
}

// Order-preserving key of an fp32 (total order for finite and inf), as
// tools/glm_model_q4k_ref.py:684-688.
__device__ __forceinline__ uint32_t f32_order_key(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u >> 31) == 0u ? (u ^ 0x80000000u) : ~u;
}

}  // namespace aipu
