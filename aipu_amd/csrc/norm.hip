// Pre-FFN RMSNorm and the residual add around the MoE step (the FFN half of
// decoder_block, tools/glm_model_q4k_ref.py:797-810, with rmsnorm :451-465).
//
//   inv  = fp32_rsqrt(f32(f32(sumsq * recip(n)) + 1e-5)),  sumsq = sequential fp32 sum of x^2
//   y[i] = bf16(f32(f32(x[i] * inv) * gamma[i]))
//   out  = bf16(f32(h[i] + fbuf[i]))                                   (residual)
//
// Reference order (AIPU_MODE_REF): the squares (exact: a bf16 squared fits fp32) go to LDS
// and one lane adds them in element order, as the LANES=1 rmsnorm_unit does; bit-exact.
// Fast mode sums them as a tree (tolerance mode, one workgroup, no serial chain).
#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"
#include "norm.hpp"

namespace aipu {
namespace {

constexpr int kNormThreads = 256;
constexpr int kSqChunk = 4096;                  // squares staged per round (16 KB)

__device__ __forceinline__ void norm_apply(const uint16_t* __restrict__ x, const uint16_t* __restrict__ gamma,
                                           int64_t n, float inv, uint16_t* __restrict__ y) {
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float xs = bf16_to_f32(x[i]) * inv;
        y[i] = (uint16_t)bf16_rne(xs * bf16_to_f32(gamma[i]));
    }
}

// Reference order: lane 0 adds the squares in element order.
__global__ void __launch_bounds__(kNormThreads) k_rmsnorm_seq(const uint16_t* __restrict__ x,
                                                              const uint16_t* __restrict__ gamma, int64_t n,
                                                              uint32_t inv_len_bits, uint16_t* __restrict__ y) {
    __shared__ __attribute__((aligned(16))) float sq[kSqChunk];
    __shared__ float s_inv;
    float s = 0.0f;
    for (int64_t base = 0; base < n; base += kSqChunk) {
        const int cnt = (int)(n - base < kSqChunk ? n - base : kSqChunk);
        for (int i = threadIdx.x; i < cnt; i += blockDim.x) {
            const float v = bf16_to_f32(x[base + i]);
            sq[i] = v * v;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            // 32 squares per batch; the next batch's LDS reads are issued before this
            // batch's adds so only the add chain is serial.
            const float4* q = reinterpret_cast<const float4*>(sq);
            const int nb = cnt / 32;
            float4 cur[8], nxt[8];
            if (nb > 0) {
#pragma unroll
                for (int j = 0; j < 8; ++j) cur[j] = q[j];
            }
            for (int b = 0; b < nb; ++b) {
                if (b + 1 < nb) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) nxt[j] = q[(b + 1) * 8 + j];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    s = s + cur[j].x;
                    s = s + cur[j].y;
                    s = s + cur[j].z;
                    s = s + cur[j].w;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) cur[j] = nxt[j];
            }
            for (int i = nb * 32; i < cnt; ++i) s = s + sq[i];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) s_inv = norm_inv(s, inv_len_bits);
    __syncthreads();
    norm_apply(x, gamma, n, s_inv, y);
}

// Tolerance mode, n <= 8 * 1024 with n % 8 == 0 and 16-B aligned vectors: each thread
// holds 8 elements of x and gamma in registers across the tree reduction (norm.hpp's order;
// the Q4_K router GEMV of the FFN half evaluates the same one, gemv_persist.hip).
constexpr int kTreeThreads = 64 * kNormWaves;

__global__ void __launch_bounds__(kTreeThreads) k_rmsnorm_vec(const uint4* __restrict__ x,
                                                              const uint4* __restrict__ gamma, int n8,
                                                              uint32_t inv_len_bits, uint4* __restrict__ y) {
    __shared__ float part[kNormWaves];
    __shared__ float s_inv;
    const int t = threadIdx.x;
    uint4 xv = make_uint4(0, 0, 0, 0), gv = make_uint4(0, 0, 0, 0);
    if (t < n8) {
        xv = x[t];
        gv = gamma[t];
    }
    const float s = norm_wave_sum(norm_sq8(xv));
    if ((t & 63) == 0) part[t >> 6] = s;
    __syncthreads();
    if (t < 64) {
        const float v = norm_final_sum(t < kNormWaves ? part[t] : 0.0f);
        if (t == 0) s_inv = norm_inv(v, inv_len_bits);
    }
    __syncthreads();
    if (t >= n8) return;
    y[t] = norm_apply8(xv, gv, s_inv);
}

// Tolerance mode, any n: per-thread strided sums, then a tree over the workgroup.
__global__ void __launch_bounds__(kTreeThreads) k_rmsnorm_tree(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ gamma, int64_t n,
                                                               uint32_t inv_len_bits, uint16_t* __restrict__ y) {
    __shared__ float part[kTreeThreads / 64];
    __shared__ float s_inv;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = bf16_to_f32(x[i]);
        s = __builtin_fmaf(v, v, s);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += shfl_xor_f(s, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int w = 0; w < kTreeThreads / 64; ++w) t += part[w];
        s_inv = norm_inv(t, inv_len_bits);
    }
    __syncthreads();
    norm_apply(x, gamma, n, s_inv, y);
}

// out may alias f (in-place residual): each element is read and written by one thread.
__global__ void k_residual_add(const uint16_t* __restrict__ h, const uint16_t* f, int64_t n, uint16_t* out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (uint16_t)bf16_rne(bf16_to_f32(h[i]) + bf16_to_f32(f[i]));
}

}  // namespace

// recip_fp32(n) of the rmsnorm unit (tools/glm_model_q4k_ref.py:434-449): q = 2^60 / n
// (floor), normalised to bit 63, 23 mantissa bits, guard = next bit, sticky = any lower bit
// of q, round half to even; a mantissa carry shifts right and bumps the exponent.
uint32_t recip_fp32_bits(int64_t n) {
    const uint64_t q = (1ull << 60) / (uint64_t)n;
    const int msb = 63 - __builtin_clzll(q);
    int expo = (msb - 60) + 127;
    const uint64_t qs = q << (63 - msb);
    uint64_t mant = (qs >> 40) & 0x7FFFFFull;
    const uint64_t guard = (qs >> 39) & 1ull;
    const uint64_t sticky = (qs & ((1ull << 39) - 1)) ? 1ull : 0ull;
    mant += guard & (sticky | (mant & 1ull));
    if (mant >> 23) {
        mant >>= 1;
        expo += 1;
    }
    return ((uint32_t)(expo & 0xFF) << 23) | (uint32_t)(mant & 0x7FFFFFull);
}

hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* gamma, int64_t n, uint16_t* y, int mode,
                          hipStream_t st) {
    const uint32_t il = recip_fp32_bits(n);
    const bool vec = n % 8 == 0 && n <= 8 * kTreeThreads && ((uintptr_t)x | (uintptr_t)gamma | (uintptr_t)y) % 16 == 0;
    if (mode == AIPU_MODE_REF)
        hipLaunchKernelGGL(k_rmsnorm_seq, dim3(1), dim3(kNormThreads), 0, st, x, gamma, n, il, y);
    else if (vec)
        hipLaunchKernelGGL(k_rmsnorm_vec, dim3(1), dim3(kTreeThreads), 0, st, (const uint4*)x, (const uint4*)gamma,
                           (int)(n / 8), il, (uint4*)y);
    else
        hipLaunchKernelGGL(k_rmsnorm_tree, dim3(1), dim3(kTreeThreads), 0, st, x, gamma, n, il, y);
    return hipGetLastError();
}

hipError_t launch_residual_add(const uint16_t* h, const uint16_t* f, int64_t n, uint16_t* out, hipStream_t st) {
    int64_t b = (n + 255) / 256;
    b = b < 1 ? 1 : (b > 1024 ? 1024 : b);
    hipLaunchKernelGGL(k_residual_add, dim3((unsigned)b), dim3(256), 0, st, h, f, n, out);
    return hipGetLastError();
}

}  // namespace aipu
