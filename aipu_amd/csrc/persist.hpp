// Helpers of the persistent matrix-core kernels (gemv_persist.hip, moe_persist.hip): LDS
// counters that waves post and poll, the compile-time loop that unrolls the copy schedule,
// and the LDS row pitch of a copied tile.
#pragma once

#include "common.hpp"
#include "mfma_gemv.hpp"

namespace aipu {
namespace pst {

using mg::lds_addr;

// Row pitch in LDS: the row bytes rounded so that consecutive rows start 32 B apart modulo
// 256, which spreads the 8 rows' reads of one column over different banks.
__host__ __device__ constexpr uint32_t tile_pitch(uint32_t rb) { return rb + ((32u - rb % 256u) + 256u) % 256u; }

template <int N>
struct IC {
    static constexpr int value = N;
};
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(IC<B>{});
        static_for<B + 1, E>(f);
    }
}

// LDS counters.  A post is one ds_add from lane 0 (exec = 1); DS operations of a wave
// execute in order, so a post issued after a wave's LDS writes makes them visible to a wave
// that reads the counter first.  The polls wait inside the asm, so the compiler never
// orders them behind direct-to-LDS copies still in flight.
// Counter addresses are LDS byte addresses (uint32_t): a constant generic pointer cast to
// LDS inside an asm operand makes the compiler emit an invalid null check.
__device__ __forceinline__ void lds_post(uint32_t c) {
    uint64_t saved;
    asm volatile("s_mov_b64 %0, exec\n\ts_mov_b64 exec, 1\n\tds_add_u32 %1, %2\n\ts_mov_b64 exec, %0"
                 : "=&s"(saved) : "v"(c), "v"(1u) : "memory");
}
__device__ __forceinline__ void lds_post(uint32_t* c) { lds_post(lds_addr(c)); }
__device__ __forceinline__ uint32_t lds_add_rtn(uint32_t* c) {
    uint64_t saved;
    uint32_t old;
    asm volatile(
        "s_mov_b64 %1, exec\n\ts_mov_b64 exec, 1\n\tds_add_rtn_u32 %0, %2, %3\n\ts_waitcnt lgkmcnt(0)\n\ts_mov_b64 exec, %1"
        : "=&v"(old), "=&s"(saved) : "v"(lds_addr(c)), "v"(1u) : "memory");
    return __builtin_amdgcn_readfirstlane(old);
}
__device__ __forceinline__ uint32_t lds_poll(const uint32_t* c) {
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(c)) : "memory");
    return __builtin_amdgcn_readfirstlane(v);
}
// Bounded wait for a counter: every wave reaches the end of the kernel even if a post were
// lost (the result would then be wrong, never a hang).
__device__ __forceinline__ void spin_ge(const uint32_t* c, uint32_t v) {
    for (uint32_t it = 0; lds_poll(c) < v && it < (1u << 22); ++it) __builtin_amdgcn_s_sleep(1);
}
// A post that also wakes the workgroup's sleeping waves once the add has executed, and the
// wait that pairs with it: long sleeps (2048 cycles) that the wakeup cuts short, so waiting
// waves take almost no issue slots from the ones computing.  A wakeup that lands between a
// poll and the sleep costs at most one sleep.
__device__ __forceinline__ void lds_post_wake(uint32_t c) {
    lds_post(c);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_wakeup" ::: "memory");
}
__device__ __forceinline__ void wait_woken(const uint32_t* c, uint32_t v) {
    for (uint32_t it = 0; lds_poll(c) < v && it < (1u << 17); ++it) __builtin_amdgcn_s_sleep(32);
}


// ------------------------------------------------------------------ one block pair
// A set is 8 rows x 2 blocks (one pass of 8 MFMAs, v_mfma_f32_16x16x32_bf16): lane 16g + n
// holds row n & 7, block h = n >> 3 of the pair, K-group g (qs bytes 32g .. 32g+31); A rows
// 4g + h carry block h's activations on group g, so D[4g + h][n] is the sub-block sum of
// column n.  Codes, seeds and the block term are those of mfma_gemv.hpp.
constexpr uint32_t kStage = 1088;   // staged pair: 1 KB of operand entries + 16 sub-block sums

// Stage a pair of blocks (512 activations; lane's piece = 8 bf16 of block lane >> 5, K-group
// (lane >> 3) & 3, MFMA lane & 7) at st: operand entries in MFMA order, then the sums.
__device__ __forceinline__ void stage_pair(const uint4& xv, uint8_t* st, int lane) {
    float* sS = (float*)(st + 1024u);
    const uint32_t ones = 0x3F803F80u;
    float sm = 0.f;
    sm = mg::dot2(xv.x, ones, sm);
    sm = mg::dot2(xv.y, ones, sm);
    sm = mg::dot2(xv.z, ones, sm);
    sm = mg::dot2(xv.w, ones, sm);
    sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
    sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x4E, 0xF, 0xF, false));
    const int hh = lane >> 5, gg = (lane >> 3) & 3, tt = lane & 7;
    *(u32x4_t*)(st + 16u * (uint32_t)((tt * 4 + gg) * 2 + hh)) = mg::act_perm(xv);
    if ((lane & 3) == 0) sS[(gg * 2 + hh) * 2 + ((lane >> 2) & 1)] = sm;
}

// A staged pair's operands on the diagonal lanes (16g + 4g + h, h < 2; every other lane keeps
// its zeros) and lane 16g + n's sub-block sums (block n >> 3, group g).
__device__ __forceinline__ void read_pair_operands(u32x4_t (&A)[8], float2& as, uint32_t st, int g, int n) {
    const uint32_t aa = st + 32u * (uint32_t)g + 16u * (uint32_t)((n - 4 * g) & 1);
    const uint32_t sa = st + 1024u + 8u * (uint32_t)(g * 2 + (n >> 3));
    uint64_t saved;
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n\t"
        "s_mov_b64 %[sv], exec\n\t"
        "s_and_b64 exec, exec, %[mask]\n\t"
        "ds_read_b128 %[a0], %[aa]\n\t"
        "ds_read_b128 %[a1], %[aa] offset:128\n\t"
        "ds_read_b128 %[a2], %[aa] offset:256\n\t"
        "ds_read_b128 %[a3], %[aa] offset:384\n\t"
        "ds_read_b128 %[a4], %[aa] offset:512\n\t"
        "ds_read_b128 %[a5], %[aa] offset:640\n\t"
        "ds_read_b128 %[a6], %[aa] offset:768\n\t"
        "ds_read_b128 %[a7], %[aa] offset:896\n\t"
        "s_mov_b64 exec, %[sv]\n\t"
        "ds_read_b64 %[as], %[sa]\n\t"
        "s_waitcnt lgkmcnt(0)"
        : [a0] "+v"(A[0]), [a1] "+v"(A[1]), [a2] "+v"(A[2]), [a3] "+v"(A[3]), [a4] "+v"(A[4]), [a5] "+v"(A[5]),
          [a6] "+v"(A[6]), [a7] "+v"(A[7]), [as] "=&v"(as), [sv] "=&s"(saved)
        : [aa] "v"(aa), [mask] "s"(mg::diag_mask(2)), [sa] "v"(sa)
        : "memory", "scc");   // s_and_b64 writes SCC
}

// The block term (block_sum of the K-group terms) of column n from its weights (header hv,
// qs dwords q0, q1 of group g) and the pair's operands.
__device__ __forceinline__ float pair_block_term(const u32x4_t (&A)[8], float2 as, const u32x4_t& hv,
                                                 const u32x4_t& q0, const u32x4_t& q1, const mg::HdrSel& hs,
                                                 const mg::CodeK& ck, int h) {
    mg::f32x4_t dlo, dhi;
    dlo[0] = dlo[1] = -mg::kCodeBiasF * as.x;
    dhi[0] = dhi[1] = -mg::kCodeBiasF * as.y;
    dlo[2] = dlo[3] = dhi[2] = dhi[3] = 0.f;
    const uint32_t qd[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        dlo = mg::mfma(A[tt], mg::codes_lo(qd[2 * tt], qd[2 * tt + 1], ck), dlo);
        dhi = mg::mfma(A[4 + tt], mg::codes_hi(qd[2 * tt], qd[2 * tt + 1], ck), dhi);
    }
    const mg::Hdr H = mg::hdr_decode(make_uint4(hv.x, hv.y, hv.z, hv.w), hs);
    return mg::block_sum(mg::block_term(H, h ? dlo[1] : dlo[0], h ? dhi[1] : dhi[0], as.x, as.y));
}

// The fast-mode tree over the pair sums of one 8-row tile: rt[row * stride + p], p < np, on
// lane 8 * row + k; every lane of a row's group of eight ends with the row's sum.
__device__ __forceinline__ float tile_tree(const float* rt, int stride, int np, int lane) {
    const int rr = lane >> 3, k = lane & 7;
    float v = k < np ? rt[rr * stride + k] : 0.0f;
    for (int j = k + 8; j < np; j += 8) v += rt[rr * stride + j];
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    return v;
}

}  // namespace pst
}  // namespace aipu
