// Shared device helpers for the gfx950 Q4_K GEMM core.
//
// The whole library is compiled with -ffp-contract=off: every `a * b + c` written in
// plain C++ is two correctly rounded fp32 ops, exactly as numpy evaluates the reference
// (tools/q4k_ref.py:53-59,91).  Fast kernels that want a fused multiply-add say so with
// __builtin_fmaf.  fp32 and fp16 denormals stay enabled (no flush-to-zero flags).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace aipu {

constexpr int QK_K = 256;

enum : int { T_F16 = 1, T_Q8_0 = 8, T_Q4_K = 12, T_Q6_K = 14, T_BF16 = 30 };

// Block geometry: weights per block, bytes per block.
__host__ __device__ constexpr int type_qk(int t) {
    return t == T_Q4_K || t == T_Q6_K ? 256 : t == T_Q8_0 ? 32 : 1;
}
__host__ __device__ constexpr int type_bytes(int t) {
    return t == T_Q4_K ? 144 : t == T_Q6_K ? 210 : t == T_Q8_0 ? 34 : 2;
}
__host__ __device__ constexpr int64_t row_bytes(int t, int64_t K) { return K / type_qk(t) * type_bytes(t); }

// ---------------------------------------------------------------- fp conversions
// Exact IEEE half -> single (v_cvt_f32_f16 with fp16 denormals enabled).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)(h & 0xFFFFu)));
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round-to-nearest-even; inf/nan keep their top 16 bits (truncation),
// the reference's rule in tools/q4k_ref.py:76-84.
__device__ __forceinline__ uint32_t bf16_rne(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7F800000u) == 0x7F800000u) return u >> 16;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// ------------------------------------------------------------ Q4_K scale unpack
// ggml get_scale_min_k4 (tools/q4k_ref.py:27-37) on the 12 packed bytes held in three
// little-endian dwords s0 = bytes 0..3, s1 = bytes 4..7, s2 = bytes 8..11.
__device__ __forceinline__ void q4k_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2,
                                              uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63u;
        m = (s1 >> (8 * j)) & 63u;
    } else {
        const int jj = j - 4;
        const uint32_t b8 = (s2 >> (8 * jj)) & 0xFFu;       // scales[j+4]
        sc = (b8 & 0x0Fu) | (((s0 >> (8 * jj + 6)) & 3u) << 4);   // top bits of scales[j-4]
        m = (b8 >> 4) | (((s1 >> (8 * jj + 6)) & 3u) << 4);       // top bits of scales[j]
    }
}

// ------------------------------------------------------- exact per-weight dequant
// Q4_K weight k (0..255) of one block at byte pointer b (any alignment; byte reads).
// w = f32(f32(d*sc)*q) - f32(dmin*m)   (tools/q4k_ref.py:53-59)
__device__ __forceinline__ float q4k_weight_exact(float D, float Mn, uint32_t q) {
    float p = D * (float)q;
    return p - Mn;
}

// ------------------------------------------------------------ buffer loads
// Raw buffer loads through a buffer resource of `bytes` bytes: an access at or beyond
// `bytes` returns 0 instead of touching memory.  Used where a load must be issued
// unconditionally (so the compiler neither branches around it nor waits for unrelated
// earlier loads where branches join) but may fall outside the data.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    // word 3 = 0x00020000: raw (untyped) 32-bit data format on gfx9-family parts
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0);
}

// ---------------------------------------------------------------- wave helpers
__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

}  // namespace aipu
