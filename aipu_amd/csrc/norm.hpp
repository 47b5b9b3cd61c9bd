// Pieces of the fast (tolerance-mode) pre-FFN RMSNorm shared by its own kernel (norm.hip) and
// by the router GEMV that applies it to its activation rows in the same launch
// (gemv_persist.hip).  Both evaluate one sum of squares in one order, so they produce the same
// bits (tools/glm_model_q4k_ref.py:432-465 for eps and the formula):
//   1. a lane's 8 consecutive elements (one 16-B load): s = fma(x, x, s) in element order;
//   2. a wave's 64 lanes (512 elements): butterfly xor 32, 16, ..., 1, lane 0's value;
//   3. up to 16 wave sums on lanes 0..15 (zero beyond the data): butterfly xor 8, 4, 2, 1,
//      lane 0's value;
//   inv = rsqrt(sumsq * recip(n) + 1e-5), y = bf16((x * inv) * gamma).
#pragma once

#include "common.hpp"
#include "glm_act.hpp"

namespace aipu {

constexpr uint32_t kNormEpsBits = 0x3727C5ACu;   // 1e-5, tools/glm_model_q4k_ref.py:432
constexpr int kNormWaves = 16;                    // wave sums of the fast reduction (n <= 8192)

__device__ __forceinline__ float norm_inv(float sumsq, uint32_t inv_len_bits) {
    const float mean = sumsq * __uint_as_float(inv_len_bits);
    return glm_rsqrt(mean + __uint_as_float(kNormEpsBits));
}

__device__ __forceinline__ float norm_sq8(const uint4& xv) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float a = __uint_as_float(xw[k] << 16), b = __uint_as_float(xw[k] & 0xFFFF0000u);
        s = __builtin_fmaf(a, a, s);
        s = __builtin_fmaf(b, b, s);
    }
    return s;
}

__device__ __forceinline__ float norm_wave_sum(float s) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += shfl_xor_f(s, o);
    return s;
}

__device__ __forceinline__ float norm_final_sum(float v) {
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) v += shfl_xor_f(v, o);
    return v;
}

__device__ __forceinline__ uint4 norm_apply8(const uint4& xv, const uint4& gv, float inv) {
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float lo = (__uint_as_float(xw[k] << 16) * inv) * __uint_as_float(gw[k] << 16);
        const float hi = (__uint_as_float(xw[k] & 0xFFFF0000u) * inv) * __uint_as_float(gw[k] & 0xFFFF0000u);
        o[k] = bf16_rne(lo) | (bf16_rne(hi) << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace aipu
