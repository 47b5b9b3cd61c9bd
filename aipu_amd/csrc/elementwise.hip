// Exact dequantisation, scale unpack, bf16 rounding and glm activations: bit-exact
// restatements of the reference's per-element arithmetic (none is on the decode path's
// bandwidth-critical leg), plus the read-bandwidth probe.
#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"

namespace aipu {

namespace {

constexpr int kThreads = 256;

inline int grid_for(int64_t work, int per_block = kThreads) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g > 65535 * 16) g = 65535 * 16;
    return (int)(g < 1 ? 1 : g);
}

// Q4_K: one thread per 4 consecutive weights.  Block byte layout fp16 d | fp16 dmin |
// scales[12] | qs[128] (tools/q4k_ref.py:12-16); for 64-group g the low nibbles of
// qs[32g..32g+31] are weights 64g..64g+31 (sub-block 2g), the high nibbles the next 32
// (sub-block 2g+1) (tools/q4k_ref.py:51-60).
__global__ void k_dequant_q4k(const uint8_t* __restrict__ blk, int64_t nquads, float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nquads; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = i >> 6;
        const int t = (int)(i & 63);
        const uint8_t* p = blk + b * 144;
        const uint32_t h0 = *(const uint32_t*)(p + 0);
        const uint32_t s0 = *(const uint32_t*)(p + 4);
        const uint32_t s1 = *(const uint32_t*)(p + 8);
        const uint32_t s2 = *(const uint32_t*)(p + 12);
        const int g = t >> 4;
        const int pos = 4 * (t & 15);                 // 0..60 within the 64-group
        const int hi = pos >= 32;
        const int j = 2 * g + hi;
        const uint32_t q4 = *(const uint32_t*)(p + 16 + 32 * g + (pos & 31));
        uint32_t sc, m;
        q4k_scale_min(j, s0, s1, s2, sc, m);
        const float d = f16_to_f32(h0), dm = f16_to_f32(h0 >> 16);
        const float D = d * (float)sc;                // f32(d*sc)
        const float Mn = dm * (float)m;               // f32(dmin*m)
        float* o = out + b * 256 + 64 * g + pos;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t q = (q4 >> (8 * e + 4 * hi)) & 0xFu;
            o[e] = q4k_weight_exact(D, Mn, q);
        }
    }
}

// Q6_K: one thread per 4 consecutive weights of a 210-B block (ql[128] qh[64] sc[16] d):
// position 128h + 32t + l takes the low (t<2) / high (t>=2) nibble of ql[64h + l + 32(t&1)]
// and bits 2t..2t+1 of qh[32h + l]; w = f32(f32(d*sc[p>>4]) * (code-32))
// (tools/q4k_ref.py:112-123).
__global__ void k_dequant_q6k(const uint8_t* __restrict__ blk, int64_t nquads, float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nquads; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = i >> 6;
        const int p0 = 4 * (int)(i & 63);
        const uint8_t* p = blk + b * 210;
        const int h = p0 >> 7, t = (p0 >> 5) & 3, l0 = p0 & 31;
        const float d = f16_to_f32((uint32_t)p[208] | ((uint32_t)p[209] << 8));
        const float ds = d * (float)(int8_t)p[192 + (p0 >> 4)];
        float* o = out + b * 256 + p0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int l = l0 + e;
            const uint32_t qlb = p[64 * h + l + 32 * (t & 1)];
            const uint32_t nib = t < 2 ? (qlb & 0xFu) : (qlb >> 4);
            const uint32_t code = nib | (((uint32_t)(p[128 + 32 * h + l] >> (2 * t)) & 3u) << 4);
            o[e] = ds * (float)((int)code - 32);
        }
    }
}

// Q8_0: 34-B blocks fp16 d | int8 qs[32]; w = f32(d * qs)  (tools/q4k_ref.py:126-129).
__global__ void k_dequant_q8_0(const uint8_t* __restrict__ blk, int64_t nquads, float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nquads; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = i >> 3;
        const int q0 = 4 * (int)(i & 7);
        const uint8_t* p = blk + b * 34;
        const float d = f16_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8));
        float* o = out + b * 32 + q0;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = d * (float)(int8_t)p[2 + q0 + e];
    }
}

__global__ void k_dequant_16(const uint16_t* __restrict__ h, int64_t n, float* __restrict__ out, int is_bf16) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = is_bf16 ? bf16_to_f32(h[i]) : f16_to_f32(h[i]);
}

__global__ void k_scale_min(const uint8_t* __restrict__ blk, int64_t n, uint16_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n * 8; i += (int64_t)gridDim.x * blockDim.x) {
        const uint8_t* p = blk + (i >> 3) * 144;
        const uint32_t s0 = *(const uint32_t*)(p + 4);
        const uint32_t s1 = *(const uint32_t*)(p + 8);
        const uint32_t s2 = *(const uint32_t*)(p + 12);
        uint32_t sc, m;
        q4k_scale_min((int)(i & 7), s0, s1, s2, sc, m);
        out[i] = (uint16_t)(sc | (m << 8));
    }
}

__global__ void k_bf16_round(const float* __restrict__ x, int64_t n, uint16_t* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (uint16_t)bf16_rne(x[i]);
}

__global__ void k_act(const uint16_t* __restrict__ x, int64_t n, uint16_t* __restrict__ y, int which) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = (uint16_t)(which == 0 ? glm_silu_bf16(x[i]) : glm_sigmoid_bf16(x[i]));
}

__global__ void k_rsqrt(const float* __restrict__ x, int64_t n, float* __restrict__ y) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = glm_rsqrt(x[i]);
}

// Read-bandwidth probe: each thread issues 8 independent 16-B loads (a 32 KB tile per
// 256-thread workgroup, coalesced) before folding them, grid-striding over the buffer.
// The fold is stored only when it equals `magic` (practically never), so the probe
// measures reads without a write or atomic stream behind it.
__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ p, int64_t n16, uint32_t* sink,
                                                     uint32_t magic) {
    uint32_t acc = 0;
    const int64_t tile = 256 * 8;
    for (int64_t base = (int64_t)blockIdx.x * tile; base < n16; base += (int64_t)gridDim.x * tile) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t i = base + u * 256 + threadIdx.x;
            v[u] = i < n16 ? p[i] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == magic) sink[blockIdx.x & 255] = acc;
}

}  // namespace

hipError_t launch_stream_read(const void* p, int64_t bytes, uint32_t* sink, hipStream_t st) {
    const int64_t n16 = bytes / 16;
    int64_t g = (n16 + 256 * 8 - 1) / (256 * 8);
    if (g > 256 * 16) g = 256 * 16;
    if (g < 1) g = 1;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)g), dim3(256), 0, st, (const uint4*)p, n16, sink, 0x9E3779B9u);
    return hipGetLastError();
}

hipError_t launch_dequant(int type, const void* blocks, int64_t n_weights, float* out, hipStream_t st) {
    const uint8_t* b = (const uint8_t*)blocks;
    switch (type) {
        case T_Q4_K: {
            const int64_t nq = n_weights / 4;
            hipLaunchKernelGGL(k_dequant_q4k, dim3(grid_for(nq)), dim3(kThreads), 0, st, b, nq, out);
            break;
        }
        case T_Q6_K: {
            const int64_t nq = n_weights / 4;
            hipLaunchKernelGGL(k_dequant_q6k, dim3(grid_for(nq)), dim3(kThreads), 0, st, b, nq, out);
            break;
        }
        case T_Q8_0: {
            const int64_t nq = n_weights / 4;
            hipLaunchKernelGGL(k_dequant_q8_0, dim3(grid_for(nq)), dim3(kThreads), 0, st, b, nq, out);
            break;
        }
        case T_F16:
        case T_BF16:
            hipLaunchKernelGGL(k_dequant_16, dim3(grid_for(n_weights)), dim3(kThreads), 0, st, (const uint16_t*)blocks,
                               n_weights, out, type == T_BF16 ? 1 : 0);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_q4k_scale_min(const void* blocks, int64_t n_blocks, uint16_t* out, hipStream_t st) {
    hipLaunchKernelGGL(k_scale_min, dim3(grid_for(n_blocks * 8)), dim3(kThreads), 0, st, (const uint8_t*)blocks,
                       n_blocks, out);
    return hipGetLastError();
}

hipError_t launch_bf16_round(const float* x, int64_t n, uint16_t* out, hipStream_t st) {
    hipLaunchKernelGGL(k_bf16_round, dim3(grid_for(n)), dim3(kThreads), 0, st, x, n, out);
    return hipGetLastError();
}

hipError_t launch_act(int which, const uint16_t* x, int64_t n, uint16_t* y, hipStream_t st) {
    hipLaunchKernelGGL(k_act, dim3(grid_for(n)), dim3(kThreads), 0, st, x, n, y, which);
    return hipGetLastError();
}

hipError_t launch_rsqrt(const float* x, int64_t n, float* y, hipStream_t st) {
    hipLaunchKernelGGL(k_rsqrt, dim3(grid_for(n)), dim3(kThreads), 0, st, x, n, y);
    return hipGetLastError();
}

}  // namespace aipu
