// MoE router: the bf16 router GEMV (logits only) and the standalone router tail.
//
// The routing decision itself (route.hpp) follows tools/glm_model_q4k_ref.py:663-699.  The
// fast MoE step computes it inside the gate/up kernel from the logits (every workgroup
// routes for itself, so no workgroup has to wait for another one); the tail kernel here
// serves the reference path, large expert counts and aipu_router_topk.
#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"
#include "route.hpp"

namespace aipu {

namespace {

constexpr int kMaxE = 4096;
constexpr int kMaxTopk = 32;

// One wave runs the tail: each round takes the largest remaining key with a wave-wide max
// (E up to 4096).  keys: LDS scratch of E entries.
__device__ void router_tail_wave(const uint16_t* logits, int E, int topk, uint32_t scale_bits, int32_t* sel,
                                 uint16_t* selw, int32_t* sel2, uint16_t* selw2, uint16_t* gates_out,
                                 uint32_t* keys, uint32_t* win) {
    const int lane = threadIdx.x & 63;
    for (int e = lane; e < E; e += 64) {
        const uint32_t lb = logits[e];
        if (gates_out) gates_out[e] = (uint16_t)glm_sigmoid_bf16(lb);
        keys[e] = route_key(lb, e);
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
        route_weights(win, topk, scale_bits, sel, selw);
        if (sel2 || selw2)
            for (int i = 0; i < topk; ++i) {
                if (sel2) sel2[i] = sel[i];
                if (selw2) selw2[i] = selw[i];
            }
    }
}

__global__ __launch_bounds__(64) void k_router_tail(const uint16_t* __restrict__ logits, int E, int topk,
                                                    uint32_t scale_bits, int32_t* sel, uint16_t* selw,
                                                    uint16_t* gates, int32_t* sel2, uint16_t* selw2) {
    __shared__ uint32_t keys[kMaxE];
    __shared__ uint32_t win[kMaxTopk];
    router_tail_wave(logits, E, topk, scale_bits, sel, selw, sel2, selw2, gates, keys, win);
}

// One routing decision per activation row (row = workgroup), E <= kRouteMaxE: every thread
// forms one key and one wave takes the top-k (route.hpp), the same decision as the one-wave
// tail.
constexpr int kRankThreads = 2 * kRouteMaxE;

__global__ __launch_bounds__(kRankThreads) void k_router_rank_rows(const uint16_t* __restrict__ logits, int E,
                                                                   int topk, uint32_t scale_bits, int32_t* sel,
                                                                   uint16_t* selw, int32_t* sel2, uint16_t* selw2) {
    __shared__ __align__(16) uint32_t keys[kRouteMaxE];
    __shared__ uint32_t win[kRouteMaxTopk];
    __shared__ int32_t s_sel[kRouteMaxTopk];
    __shared__ uint16_t s_selw[kRouteMaxTopk];
    const int r = blockIdx.x, t = threadIdx.x;
    route_workgroup(logits + (int64_t)r * E, E, topk, scale_bits, keys, win, s_sel, s_selw, true);
    if (t < topk) {
        sel[r * topk + t] = s_sel[t];
        selw[r * topk + t] = s_selw[t];
        if (sel2) sel2[r * topk + t] = s_sel[t];
        if (selw2) selw2[r * topk + t] = s_selw[t];
    }
}

// One routing decision per activation row (row = workgroup), any E <= kMaxE.
__global__ __launch_bounds__(64) void k_router_tail_rows(const uint16_t* __restrict__ logits, int E, int topk,
                                                         uint32_t scale_bits, int32_t* sel, uint16_t* selw,
                                                         int32_t* sel2, uint16_t* selw2) {
    __shared__ uint32_t keys[kMaxE];
    __shared__ uint32_t win[kMaxTopk];
    const int r = blockIdx.x;
    router_tail_wave(logits + (int64_t)r * E, E, topk, scale_bits, sel + r * topk, selw + r * topk,
                     sel2 ? sel2 + r * topk : nullptr, selw2 ? selw2 + r * topk : nullptr, nullptr, keys, win);
}

// bf16 router GEMV: workgroup e computes logit e (256 threads split K; fixed-order
// reduction) and writes it as bf16.

__global__ __launch_bounds__(kRouterThreads) void k_router_logits(const uint16_t* __restrict__ W,
                                                                  const uint16_t* __restrict__ x, int64_t K,
                                                                  uint16_t* __restrict__ logits) {
    __shared__ float wsum[kRouterThreads / 64];
    const int t = threadIdx.x, e = blockIdx.x;
    const float v = router_wave_dot(W + (int64_t)e * K, x, K, t);
    if ((t & 63) == 0) wsum[t >> 6] = v;
    __syncthreads();
    if (t == 0) logits[e] = (uint16_t)bf16_rne(router_logit(wsum));
}

// bf16 router GEMV for M <= 8 activation rows: workgroup e reads router row e once and forms
// logit e of every row (same per-row arithmetic as k_router_logits).
template <int MR>
__global__ __launch_bounds__(kRouterThreads) void k_router_logits_rows(const uint16_t* __restrict__ W,
                                                                       const uint16_t* __restrict__ x, int64_t K,
                                                                       int M, int E, uint16_t* __restrict__ logits) {
    __shared__ float wsum[MR][kRouterThreads / 64];
    const int t = threadIdx.x, e = blockIdx.x;
    const uint16_t* row = W + (int64_t)e * K;
    float s0[MR], s1[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) s0[m] = s1[m] = 0.f;
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    // four chunks' router loads are issued before any is used (K = 6144 is three chunks per
    // thread); each row still folds its chunks into s0 / s1 in increasing K
    constexpr int kU = 4;
    for (int64_t c0 = (int64_t)t * 8; c0 < K; c0 += kU * kRouterThreads * 8) {
        uint4 wv[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t c = c0 + (int64_t)u * kRouterThreads * 8;
            if (c < K) wv[u] = *(const uint4*)(row + c);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t c = c0 + (int64_t)u * kRouterThreads * 8;
            if (c >= K) break;
            const uint4 w = wv[u];
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                if (m >= M) break;
                const uint4 a = *(const uint4*)(x + (int64_t)m * K + c);
                s0[m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.x), __builtin_bit_cast(bf2, w.x), s0[m], false);
                s1[m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.y), __builtin_bit_cast(bf2, w.y), s1[m], false);
                s0[m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.z), __builtin_bit_cast(bf2, w.z), s0[m], false);
                s1[m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.w), __builtin_bit_cast(bf2, w.w), s1[m], false);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float v = s0[m] + s1[m];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
        if ((t & 63) == 0) wsum[m][t >> 6] = v;
    }
    __syncthreads();
    if (t < M) {
        float tot = 0.f;
        for (int w = 0; w < kRouterThreads / 64; ++w) tot += wsum[t][w];
        logits[(int64_t)t * E + e] = (uint16_t)bf16_rne(tot);
    }
}

}  // namespace

hipError_t launch_router_bf16_logits_rows(const uint16_t* W, const uint16_t* x, int64_t K, int E, int M,
                                          uint16_t* logits, hipStream_t st) {
    if (M < 1 || M > 8) return hipErrorInvalidValue;
    if (M <= 2)
        hipLaunchKernelGGL(k_router_logits_rows<2>, dim3(E), dim3(kRouterThreads), 0, st, W, x, K, M, E, logits);
    else
        hipLaunchKernelGGL(k_router_logits_rows<8>, dim3(E), dim3(kRouterThreads), 0, st, W, x, K, M, E, logits);
    return hipGetLastError();
}

hipError_t launch_router_tail(const uint16_t* logits, int E, int topk, uint32_t scale_bits, int32_t* sel_idx,
                              uint16_t* sel_w, uint16_t* gates, hipStream_t st, int32_t* sel2, uint16_t* selw2) {
    hipLaunchKernelGGL(k_router_tail, dim3(1), dim3(64), 0, st, logits, E, topk, scale_bits, sel_idx, sel_w, gates,
                       sel2, selw2);
    return hipGetLastError();
}

hipError_t launch_router_tail_rows(const uint16_t* logits, int M, int E, int topk, uint32_t scale_bits, int32_t* sel,
                                   uint16_t* selw, int32_t* sel2, uint16_t* selw2, hipStream_t st) {
    if (E <= kRouteMaxE && topk <= kRouteMaxTopk) {
        hipLaunchKernelGGL(k_router_rank_rows, dim3(M), dim3(kRankThreads), 0, st, logits, E, topk, scale_bits, sel, selw,
                           sel2, selw2);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_router_tail_rows, dim3(M), dim3(64), 0, st, logits, E, topk, scale_bits, sel, selw, sel2,
                       selw2);
    return hipGetLastError();
}

hipError_t launch_router_bf16_logits(const uint16_t* W, const uint16_t* x, int64_t K, int E, uint16_t* logits,
                                     hipStream_t st) {
    hipLaunchKernelGGL(k_router_logits, dim3(E), dim3(kRouterThreads), 0, st, W, x, K, logits);
    return hipGetLastError();
}

}  // namespace aipu
