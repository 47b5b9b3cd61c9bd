// MoE routing decision shared by the router tail kernel and the in-kernel routing of the
// gate/up leg (tools/glm_model_q4k_ref.py:663-699):
//   gate = glm_sigmoid(logit) (bf16); experts ordered by (fp32 order key of the gate,
//   descending; expert index, ascending); the first topk win; s = balanced +0-padded fp32
//   add tree over the winners' gates in slot order; rs = f32(f32(rsqrt(s)^2) * SCALE);
//   sel_w = bf16(gate * rs).
// Because the gates are bf16, the fp32 order key of a gate is the 16-bit order key of its
// bf16 pattern followed by 16 zero bits, so one 32-bit key (key16 << 16 | 0xFFFF - e)
// orders experts exactly as the reference's (key, -e) sort, ties included, and all keys
// are distinct.
#pragma once

#include "common.hpp"
#include "glm_act.hpp"

namespace aipu {

constexpr int kRouteMaxE = 512;    // in-kernel routing (one key per thread, eight per lane of the top-k wave)
constexpr int kRouteMaxTopk = 32;

__device__ __forceinline__ uint32_t bf16_order_key(uint32_t b) {
    return (b & 0x8000u) ? (~b & 0xFFFFu) : (b ^ 0x8000u);
}

__device__ __forceinline__ uint32_t key_to_bf16(uint32_t k16) {
    return (k16 & 0x8000u) ? (k16 ^ 0x8000u) : (~k16 & 0xFFFFu);
}

__device__ __forceinline__ uint32_t route_key(uint32_t logit_bits, int e) {
    return (bf16_order_key(glm_sigmoid_bf16(logit_bits)) << 16) | (0xFFFFu - (uint32_t)e);
}

// Slot weights from the winners' keys in slot order (one thread): the balanced fp32 add
// tree over the gates (padded with +0 to a power of two >= 2), rs = rsqrt(s)^2 * scale.
// The tree is written with compile-time trip counts so the nodes stay in registers.
__device__ __forceinline__ void route_weights(const uint32_t* win, int topk, uint32_t scale_bits, int32_t* sel,
                                              uint16_t* selw) {
    float node[kRouteMaxTopk];
#pragma unroll
    for (int i = 0; i < kRouteMaxTopk; ++i) node[i] = i < topk ? bf16_to_f32(key_to_bf16(win[i] >> 16)) : 0.0f;
    int npow = 2;
    while (npow < topk) npow <<= 1;
#pragma unroll
    for (int n = kRouteMaxTopk; n > 1; n >>= 1) {
        if (n <= npow) {
#pragma unroll
            for (int i = 0; i < n / 2; ++i) node[i] = node[2 * i] + node[2 * i + 1];
        }
    }
    const float rr = glm_rsqrt(node[0]);
    const float rr2 = rr * rr;
    const float rs = rr2 * __uint_as_float(scale_bits);
    for (int i = 0; i < topk; ++i) {
        const float g = bf16_to_f32(key_to_bf16(win[i] >> 16));
        sel[i] = (int32_t)(0xFFFFu - (win[i] & 0xFFFFu));
        selw[i] = (uint16_t)bf16_rne(g * rs);
    }
}

// bf16 router dot product of one row (the reference's logit linear, tools/glm_model_q4k_ref.py:663-668)
// as the kRouterThreads threads of a router workgroup form it: thread t folds its 16-B chunks
// c = 8t + 2048u (u = 0, 1, ...) into two fp32 partials (dwords 0, 2 into s0; 1, 3 into s1) in
// increasing K and returns s0 + s1 summed over its wave (xor 32, 16, ..., 1); router_logit adds
// the four waves' sums in wave order.  Every kernel that forms router logits uses this order.
constexpr int kRouterThreads = 256;
__device__ __forceinline__ float router_wave_dot(const uint16_t* row, const uint16_t* x, int64_t K, int t) {
    float s0 = 0.f, s1 = 0.f;
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    // four chunks' loads are issued before any is used (K = 6144 is three chunks per thread)
    constexpr int kU = 4;
    for (int64_t c0 = (int64_t)t * 8; c0 < K; c0 += kU * kRouterThreads * 8) {
        uint4 wv[kU], av[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t c = c0 + (int64_t)u * kRouterThreads * 8;
            if (c < K) {
                wv[u] = *(const uint4*)(row + c);
                av[u] = *(const uint4*)(x + c);
            }
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t c = c0 + (int64_t)u * kRouterThreads * 8;
            if (c >= K) break;
            const uint4 w = wv[u], a = av[u];
            s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.x), __builtin_bit_cast(bf2, w.x), s0, false);
            s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.y), __builtin_bit_cast(bf2, w.y), s1, false);
            s0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.z), __builtin_bit_cast(bf2, w.z), s0, false);
            s1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a.w), __builtin_bit_cast(bf2, w.w), s1, false);
        }
    }
    float v = s0 + s1;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float router_logit(const float* wsum) {
    float tot = 0.f;
    for (int w = 0; w < kRouterThreads / 64; ++w) tot += wsum[w];
    return tot;
}

// Largest value over the wave (DPP: prefix maxima within each row of 16 lanes, then rows 0-1 and
// 0-3 meet in lanes 31 and 63).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x111, 0xF, 0xF, false));   // row_shr:1
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x112, 0xF, 0xF, false));   // row_shr:2
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x114, 0xF, 0xF, false));   // row_shr:4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x118, 0xF, 0xF, false));   // row_shr:8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));   // row_bcast:15
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));   // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
}

// The winners of one row by one wave (all 64 lanes): lane l holds keys k[j] of experts
// l + 64j (0 past E, below every key), and topk rounds each take the largest remaining key, so
// win[0..topk) comes out in slot order (keys are distinct: one lane and register hold each).
constexpr int kRouteKeysPerLane = kRouteMaxE / 64;
__device__ __forceinline__ void route_tournament(uint32_t (&k)[kRouteKeysPerLane], int topk, uint32_t* win, int lane) {
    for (int i = 0; i < topk; ++i) {
        uint32_t head = k[0];
#pragma unroll
        for (int j = 1; j < kRouteKeysPerLane; ++j) head = max(head, k[j]);
        const uint32_t m = wave_max_u32(head);
#pragma unroll
        for (int j = 0; j < kRouteKeysPerLane; ++j) k[j] = k[j] == m ? 0u : k[j];
        if (lane == 0) win[i] = m;
    }
}

// route_tournament with the winners left one per lane: lane i < topk returns win[i].
__device__ __forceinline__ uint32_t route_tournament_lanes(uint32_t (&k)[kRouteKeysPerLane], int topk, int lane) {
    uint32_t mine = 0;
    for (int i = 0; i < topk; ++i) {
        uint32_t head = k[0];
#pragma unroll
        for (int j = 1; j < kRouteKeysPerLane; ++j) head = max(head, k[j]);
        const uint32_t m = wave_max_u32(head);
#pragma unroll
        for (int j = 0; j < kRouteKeysPerLane; ++j) k[j] = k[j] == m ? 0u : k[j];
        mine = lane == i ? m : mine;
    }
    return mine;
}

// route_weights with lane i < topk holding win[i]: the balanced +0-padded add tree over the
// gates runs as DPP row shifts (level l adds lane x - 2^(l-1) into lane x; lane 2^l (j + 1) - 1
// then holds node j of level l, since fp32 addition is commutative the bits are the serial
// tree's), rs = rsqrt(s)^2 * scale from lane npow - 1, and every lane forms its own slot.
__device__ __forceinline__ void route_weights_wave(uint32_t win_lane, int topk, uint32_t scale_bits, int lane,
                                                   int32_t& sel, uint16_t& selw) {
    const float g = bf16_to_f32(key_to_bf16(win_lane >> 16));
    float v = lane < topk ? g : 0.0f;
    int npow = 2;
    while (npow < topk) npow <<= 1;
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xF, 0xF, false));   // row_shr:1
    if (npow >= 4) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xF, 0xF, false));
    if (npow >= 8) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xF, 0xF, false));
    if (npow >= 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xF, 0xF, false));
    if (npow >= 32) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    const float s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), npow - 1));
    const float rr = glm_rsqrt(s);
    const float rr2 = rr * rr;
    const float rs = rr2 * __uint_as_float(scale_bits);
    sel = (int32_t)(0xFFFFu - (win_lane & 0xFFFFu));
    selw = (uint16_t)bf16_rne(g * rs);
}

// The routing decision computed by one workgroup (all threads call it; E <= kRouteMaxE and
// E rounded up to 8 <= the thread count, topk <= kRouteMaxTopk; keys holds >= that many).
// Every thread forms one key; wave 0 takes the top-k (route_tournament_lanes), so
// win[0..topk) holds the winners' keys in slot order; with `weights`, the wave also fills
// sel / selw (LDS, route_weights_wave).
__device__ __forceinline__ void route_workgroup(const uint16_t* logits, int E, int topk, uint32_t scale_bits,
                                                uint32_t* keys, uint32_t* win, int32_t* sel, uint16_t* selw,
                                                bool weights) {
    const int t = threadIdx.x;
    if (t < E) keys[t] = route_key(logits[t], t);
    __syncthreads();
    if (t < 64) {
        uint32_t k[kRouteKeysPerLane];
#pragma unroll
        for (int j = 0; j < kRouteKeysPerLane; ++j) k[j] = t + 64 * j < E ? keys[t + 64 * j] : 0u;
        const uint32_t wl = route_tournament_lanes(k, topk, t);
        if (t < topk) win[t] = wl;
        if (weights) {
            int32_t sl;
            uint16_t swl;
            route_weights_wave(wl, topk, scale_bits, t, sl, swl);
            if (t < topk) {
                sel[t] = sl;
                selw[t] = swl;
            }
        }
    }
    __syncthreads();
}

}  // namespace aipu
