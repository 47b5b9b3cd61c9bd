// MoE router: bf16 router GEMV fused with the router tail, and the standalone tail.
//
// Tail semantics (tools/glm_model_q4k_ref.py:663-699): gate = glm_sigmoid(logit) (bf16);
// experts ordered by (fp32 order key of the gate, descending; expert index, ascending);
// the first topk win; s = balanced +0-padded fp32 add tree over the winners in slot order;
// rs = f32(f32(rsqrt(s)^2) * SCALE); sel_w = bf16(gate * rs).
//
// Because the gates are bf16, the fp32 order key of a gate is the 16-bit order key of its
// bf16 pattern followed by 16 zero bits, so one 32-bit key (key16 << 16 | 0xFFFF - e)
// orders experts exactly as the reference's (key, -e) sort, ties included.  A single
// wave finds each winner with a wave-wide max; no workgroup barriers are needed.
#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"

namespace aipu {

namespace {

__device__ __forceinline__ uint32_t bf16_order_key(uint32_t b) {
    return (b & 0x8000u) ? (~b & 0xFFFFu) : (b ^ 0x8000u);
}

__device__ __forceinline__ uint32_t key_to_bf16(uint32_t k16) {
    return (k16 & 0x8000u) ? (k16 ^ 0x8000u) : (~k16 & 0xFFFFu);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// Coherent read of a value another workgroup wrote in this kernel (bypasses the
// non-coherent per-CU cache).
__device__ __forceinline__ uint32_t load_coherent_u16(const uint16_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr int kMaxE = 4096;
constexpr int kMaxTopk = 32;

// One wave (lanes 0..63 of the calling workgroup) runs the tail.  keys: LDS scratch of
// E entries.  `coherent` selects coherent loads for logits written by other workgroups.
__device__ void router_tail_wave(const uint16_t* logits, int E, int topk, uint32_t scale_bits, int32_t* sel,
                                 uint16_t* selw, int32_t* sel2, uint16_t* selw2, uint16_t* gates_out,
                                 uint32_t* keys, uint32_t* win, float* node, bool coherent) {
    const int lane = threadIdx.x & 63;
    for (int e = lane; e < E; e += 64) {
        const uint32_t lb = coherent ? load_coherent_u16(logits + e) : logits[e];
        const uint32_t gb = glm_sigmoid_bf16(lb);
        if (gates_out) gates_out[e] = (uint16_t)gb;
        keys[e] = (bf16_order_key(gb) << 16) | (0xFFFFu - (uint32_t)e);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    for (int s = 0; s < topk; ++s) {
        uint32_t best = 0;
        for (int e = lane; e < E; e += 64) best = keys[e] > best ? keys[e] : best;
        best = wave_max_u32(best);
        if (lane == 0) win[s] = best;
        const int e_win = (int)(0xFFFFu - (best & 0xFFFFu));
        if ((e_win & 63) == lane) keys[e_win] = 0u;   // the owning lane retires the winner
        __builtin_amdgcn_wave_barrier();
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) {
        int npow = 2, lev = 1;
        while (npow < topk) {
            npow <<= 1;
            ++lev;
        }
        for (int i = 0; i < npow; ++i) node[i] = i < topk ? bf16_to_f32(key_to_bf16(win[i] >> 16)) : 0.0f;
        for (int l = 0; l < lev; ++l)
            for (int i = 0; i < (npow >> (l + 1)); ++i) node[i] = node[2 * i] + node[2 * i + 1];
        const float rr = glm_rsqrt(node[0]);
        const float rr2 = rr * rr;
        const float rs = rr2 * __uint_as_float(scale_bits);
        for (int i = 0; i < topk; ++i) {
            const float g = bf16_to_f32(key_to_bf16(win[i] >> 16));
            const int32_t e = (int32_t)(0xFFFFu - (win[i] & 0xFFFFu));
            const uint16_t w = (uint16_t)bf16_rne(g * rs);
            sel[i] = e;
            selw[i] = w;
            if (sel2) sel2[i] = e;
            if (selw2) selw2[i] = w;
        }
    }
}

__global__ __launch_bounds__(64) void k_router_tail(const uint16_t* __restrict__ logits, int E, int topk,
                                                    uint32_t scale_bits, int32_t* sel, uint16_t* selw,
                                                    uint16_t* gates) {
    __shared__ uint32_t keys[kMaxE];
    __shared__ uint32_t win[kMaxTopk];
    __shared__ float node[kMaxTopk];
    router_tail_wave(logits, E, topk, scale_bits, sel, selw, nullptr, nullptr, gates, keys, win, node, false);
}

// bf16 router GEMV fused with the tail: workgroup e computes logit e (256 threads split K,
// fixed-order reduction), publishes it, and the last workgroup to arrive (ticket counter
// in the caller's workspace, reset to 0 by that workgroup) runs the tail.
constexpr int kRouterThreads = 256;

__global__ __launch_bounds__(kRouterThreads) void k_router_bf16(const uint16_t* __restrict__ W,
                                                                const uint16_t* __restrict__ x, int64_t K, int E,
                                                                int topk, uint32_t scale_bits,
                                                                uint16_t* __restrict__ logits, uint32_t* counter,
                                                                int32_t* sel, uint16_t* selw, int32_t* sel2,
                                                                uint16_t* selw2) {
    __shared__ float wsum[kRouterThreads / 64];
    __shared__ int is_last;
    __shared__ uint32_t keys[kMaxE];
    __shared__ uint32_t win[kMaxTopk];
    __shared__ float node[kMaxTopk];
    const int t = threadIdx.x, e = blockIdx.x;
    const uint16_t* row = W + (int64_t)e * K;
    float s0 = 0.f, s1 = 0.f;
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    for (int64_t c = (int64_t)t * 8; c < K; c += kRouterThreads * 8) {
        const uint4 w = *(const uint4*)(row + c);
        const uint4 a = *(const uint4*)(x + c);
        s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.x), __builtin_bit_cast(bf2, w.x), s0, false);
        s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.y), __builtin_bit_cast(bf2, w.y), s1, false);
        s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.z), __builtin_bit_cast(bf2, w.z), s0, false);
        s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.w), __builtin_bit_cast(bf2, w.w), s1, false);
    }
    float v = s0 + s1;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((t & 63) == 0) wsum[t >> 6] = v;
    __syncthreads();
    if (t == 0) {
        float tot = 0.f;
        for (int w = 0; w < kRouterThreads / 64; ++w) tot += wsum[w];
        logits[e] = (uint16_t)bf16_rne(tot);
        __threadfence();
        const uint32_t ticket = atomicAdd(counter, 1u);
        is_last = ticket == (uint32_t)(E - 1);
    }
    __syncthreads();
    if (!is_last) return;
    if (t < 64) {
        __threadfence();
        router_tail_wave(logits, E, topk, scale_bits, sel, selw, sel2, selw2, nullptr, keys, win, node, true);
        if (t == 0) atomicExch(counter, 0u);
    }
}

}  // namespace

hipError_t launch_router_tail(const uint16_t* logits, int E, int topk, uint32_t scale_bits, int32_t* sel_idx,
                              uint16_t* sel_w, uint16_t* gates, hipStream_t st) {
    hipLaunchKernelGGL(k_router_tail, dim3(1), dim3(64), 0, st, logits, E, topk, scale_bits, sel_idx, sel_w, gates);
    return hipGetLastError();
}

hipError_t launch_router_bf16_fused(const uint16_t* W, const uint16_t* x, int64_t K, int E, int topk,
                                    uint32_t scale_bits, uint16_t* logits, uint32_t* counter, int32_t* sel,
                                    uint16_t* selw, int32_t* sel2, uint16_t* selw2, hipStream_t st) {
    hipLaunchKernelGGL(k_router_bf16, dim3(E), dim3(kRouterThreads), 0, st, W, x, K, E, topk, scale_bits, logits,
                       counter, sel, selw, sel2, selw2);
    return hipGetLastError();
}

}  // namespace aipu
