// Helpers of the persistent matrix-core kernels (gemv_persist.hip, gemv_persist_m.hip,
// moe_persist.hip): LDS counters that waves post and poll, the compile-time loop that unrolls
// a copy schedule, the LDS row pitch of a copied tile, the activation-pair staging, and the
// copy loop of a ring of round slots.
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

// Staging of one block pair's activations (512 bf16, 1 KB) for the block-diagonal MFMA
// operand.  The operand of MFMA t (t < 4: low nibbles, sub-block 2g; t >= 4: high nibbles,
// sub-block 2g + 1) on K-group g for block h is the 16-B chunk 32h + 8g + t of the pair; it is
// stored at entry 9t + 2g + h (kStgStride = 144 B per t), so lane L = 32h + 8g + t writes its own
// contiguously loaded chunk and the eight lanes with equal (g, h) land on eight different bank
// groups.  A reader takes MFMA t's operand at 32g + 16h + 144t.  The 16 sub-block sums follow at
// kStgSums (float, index 2(2g + h) + (t >> 2)), each ((c0 + c1) + (c2 + c3)) over its four
// chunks' sums, the order every fast-mode kernel uses.
constexpr uint32_t kStgStride = 144;
constexpr uint32_t kStgSums = 1136;
constexpr uint32_t kStgBytes = 1200;
__device__ __forceinline__ void stage_pair(const uint4& xv, uint8_t* st, int L) {
    const uint32_t ones = 0x3F803F80u;
    float c = 0.f;
    c = mg::dot2(xv.x, ones, c);
    c = mg::dot2(xv.y, ones, c);
    c = mg::dot2(xv.z, ones, c);
    c = mg::dot2(xv.w, ones, c);
    c += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0xB1, 0xF, 0xF, false));   // xor 1
    c += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x4E, 0xF, 0xF, false));   // xor 2
    const int h = L >> 5, g = (L >> 3) & 3, t = L & 7;
    *(u32x4_t*)(st + 16u * (uint32_t)(9 * t + 2 * g + h)) = mg::act_perm(xv);
    if ((L & 3) == 0) ((float*)(st + kStgSums))[(g * 2 + h) * 2 + (t >> 2)] = c;
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
// A wait that gives up (below) sets this word, one per translation unit that includes this
// header, with one vector atomic; the library reads and clears it through
// aipu_wait_timeouts(), so the wrong result such a launch leaves is reported, not silent.
[[maybe_unused]] static __device__ uint32_t g_wait_gave_up;

__device__ __forceinline__ void wait_gave_up() {
    __hip_atomic_fetch_or(&g_wait_gave_up, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Host side: this translation unit's word (nonzero = some wait gave up), then cleared.
[[maybe_unused]] static hipError_t take_wait_gave_up(uint32_t* flag) {
    hipError_t e = hipMemcpyFromSymbol(flag, HIP_SYMBOL(g_wait_gave_up), sizeof(uint32_t));
    if (e == hipSuccess && *flag) {
        const uint32_t zero = 0;
        e = hipMemcpyToSymbol(HIP_SYMBOL(g_wait_gave_up), &zero, sizeof(uint32_t));
    }
    return e;
}

// Bounded wait for a counter: every wave reaches the end of the kernel even if a post were
// lost.  The result would then be wrong, never a hang, and the give-up is recorded.
__device__ __forceinline__ void spin_ge(const uint32_t* c, uint32_t v) {
    for (uint32_t it = 0; lds_poll(c) < v; ++it) {
        if (it == (1u << 22)) {
            wait_gave_up();
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Copy wave c of CW: rounds u = c, c + CW, ... < U (LOADS loads each) into slots u % NS, at
// most Q of its own in flight.  Round u is issued once its slot is free (round u - NS read by
// its READERS readers) and posted, in order among the wave's rounds, once Q - 1 later rounds
// of the wave are in flight behind it.  With CW * Q < NS a landed round has time to be read before a copy wave
// needs its slot.  While a slot is still being read, every round of the wave but the newest
// is posted first, so no reader waits for a round that has landed; the round a copy wave
// waits on is then never the other wave's unposted newest one (that would need NS = CW).
template <int NS, int Q, int CW, int LOADS, int READERS, class Issue>
__device__ __forceinline__ void copy_ring(int c, int U, uint32_t* s_cnt, uint32_t* s_read, Issue&& issue) {
    static_assert(Q >= 2 && CW * Q <= NS && LOADS * (Q - 1) <= 63, "rounds in flight within vmcnt and the ring");
    uint32_t cnt0 = lds_addr(s_cnt);
    asm volatile("" : "+v"(cnt0));   // a runtime base (see lds_post)
    const int nr = U > c ? (U - c + CW - 1) / CW : 0;   // this wave's rounds
    int posted = 0;                                      // of this wave's rounds
    for (int i = 0; i < nr; ++i) {
        const int u = c + CW * i;
        if (u >= NS && lds_poll(&s_read[u - NS]) < (uint32_t)READERS) {
            if (posted < i - 1) {
                __builtin_amdgcn_s_waitcnt(mg::wait_vm(LOADS));
                while (posted < i - 1) lds_post(cnt0 + 4u * (uint32_t)(c + CW * posted++));
            }
            spin_ge(&s_read[u - NS], (uint32_t)READERS);
        }
        issue(u);
        if (posted <= i - (Q - 1)) {
            __builtin_amdgcn_s_waitcnt(mg::wait_vm(LOADS * (Q - 1)));
            while (posted <= i - (Q - 1)) lds_post(cnt0 + 4u * (uint32_t)(c + CW * posted++));
        }
    }
    const int left = nr - posted;   // the oldest of `left` unposted rounds has landed once LOADS * (left - 1) loads remain
    static_for<0, Q - 1>([&](auto sI) {
        constexpr int j = Q - 2 - decltype(sI)::value;
        if (j < left) {
            __builtin_amdgcn_s_waitcnt(mg::wait_vm(LOADS * j));
            lds_post(cnt0 + 4u * (uint32_t)(c + CW * posted));
            ++posted;
        }
    });
}

}  // namespace pst
}  // namespace aipu
