// Exact dequantisation, scale unpack, bf16 rounding, glm activations and the MoE router
// tail.  These are bit-exact restatements of the reference's per-element arithmetic; none
// of them is bandwidth-critical on the decode path except the router tail's latency.
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

// Read-bandwidth probe: every thread streams 16-B loads grid-stride and xor-folds them.
__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ p, int64_t n16, uint32_t* sink) {
    uint32_t acc = 0;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    if ((threadIdx.x & 63) == 0) atomicXor(&sink[blockIdx.x & 255], acc);
}

}  // namespace

hipError_t launch_stream_read(const void* p, int64_t bytes, uint32_t* sink, hipStream_t st) {
    const int64_t n16 = bytes / 16;
    int64_t g = (n16 + 256 * 8 - 1) / (256 * 8);
    if (g > 256 * 16) g = 256 * 16;
    if (g < 1) g = 1;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)g), dim3(256), 0, st, (const uint4*)p, n16, sink);
    return hipGetLastError();
}

// -------------------------------------------------------------- router tail
// One workgroup of 1024 threads.  Each thread owns experts e = tid, tid+1024, ...
// Gates are glm_sigmoid of the bf16 logits; the winner of each of the topk rounds is the
// maximum of the composite key (fp32 order key << 32 | ~index), i.e. largest gate first
// and the lower expert index on ties (tools/glm_model_q4k_ref.py:671-673).  Thread 0 then
// forms the balanced +0-padded fp32 add tree over the winners in slot order (:691-699),
// rs = f32(f32(rsqrt(s)^2) * scale) (:678-679) and sel_w = bf16(gate * rs) (:680).
constexpr int kRouterThreads = 1024;
constexpr int kRouterMaxPerThread = 4;   // E <= 4096
constexpr int kMaxTopk = 32;

__device__ __forceinline__ uint64_t u64max(uint64_t a, uint64_t b) { return a > b ? a : b; }

__global__ __launch_bounds__(kRouterThreads) void k_router_tail(const uint16_t* __restrict__ logits, int E, int topk,
                                                                 uint32_t scale_bits, int32_t* __restrict__ sel_idx,
                                                                 uint16_t* __restrict__ sel_w,
                                                                 uint16_t* __restrict__ gates_out) {
    __shared__ uint64_t wave_best[kRouterThreads / 64];
    __shared__ uint64_t winners[kMaxTopk];
    const int tid = threadIdx.x;
    uint64_t key[kRouterMaxPerThread];
#pragma unroll
    for (int r = 0; r < kRouterMaxPerThread; ++r) {
        const int e = tid + r * kRouterThreads;
        key[r] = 0;
        if (e < E) {
            const uint32_t gb = glm_sigmoid_bf16(logits[e]);
            if (gates_out) gates_out[e] = (uint16_t)gb;
            key[r] = ((uint64_t)f32_order_key(bf16_to_f32(gb)) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
        }
    }
    for (int s = 0; s < topk; ++s) {
        uint64_t best = 0;
#pragma unroll
        for (int r = 0; r < kRouterMaxPerThread; ++r) best = u64max(best, key[r]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)best, off, 64);
            const uint32_t hi = __shfl_xor((uint32_t)(best >> 32), off, 64);
            best = u64max(best, ((uint64_t)hi << 32) | lo);
        }
        if ((tid & 63) == 0) wave_best[tid >> 6] = best;
        __syncthreads();
        if (tid == 0) {
            uint64_t b = 0;
            for (int w = 0; w < kRouterThreads / 64; ++w) b = u64max(b, wave_best[w]);
            winners[s] = b;
        }
        __syncthreads();
        const uint64_t win = winners[s];
#pragma unroll
        for (int r = 0; r < kRouterMaxPerThread; ++r)
            if (key[r] == win) key[r] = 0;
        __syncthreads();
    }
    if (tid == 0) {
        float node[kMaxTopk];
        int lev = 1, npow = 2;
        while (npow < topk) { npow <<= 1; ++lev; }
        for (int i = 0; i < npow; ++i) {
            if (i < topk) {
                const uint32_t ok = (uint32_t)(winners[i] >> 32);
                node[i] = __uint_as_float((ok >> 31) ? (ok ^ 0x80000000u) : ~ok);
            } else {
                node[i] = 0.0f;
            }
        }
        for (int l = 0; l < lev; ++l) {
            for (int i = 0; i < (npow >> (l + 1)); ++i) node[i] = node[2 * i] + node[2 * i + 1];
        }
        const float rr = glm_rsqrt(node[0]);
        const float rr2 = rr * rr;
        const float rs = rr2 * __uint_as_float(scale_bits);
        for (int i = 0; i < topk; ++i) {
            const uint32_t ok = (uint32_t)(winners[i] >> 32);
            const float g = __uint_as_float((ok >> 31) ? (ok ^ 0x80000000u) : ~ok);
            sel_idx[i] = (int32_t)(0xFFFFFFFFu - (uint32_t)winners[i]);
            sel_w[i] = (uint16_t)bf16_rne(g * rs);
        }
    }
}

hipError_t launch_router_tail(const uint16_t* logits, int E, int topk, uint32_t scale_bits, int32_t* sel_idx,
                              uint16_t* sel_w, uint16_t* gates, hipStream_t st) {
    hipLaunchKernelGGL(k_router_tail, dim3(1), dim3(kRouterThreads), 0, st, logits, E, topk, scale_bits, sel_idx,
                       sel_w, gates);
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
