// Persistent matrix-core legs of the MoE decode step (tolerance mode) at the config-2 shape
// (hidden 6144, expert intermediate 2048, up to 8 routed slots + 1 shared): gate/up with the
// fused h = bf16(silu(g) * u) and in-kernel routing, then down with the slot-ordered combine.
//
// Both legs run one workgroup per CU: a copy wave streams the workgroup's 8-row tiles into LDS
// (chunk-major, rounds of 9 direct-to-LDS loads = 1152 bytes of each of the 8 rows, posted to
// LDS counters as they land, Q rounds in flight, NB tile buffers), and 12 compute waves take
// 8-row x 2-block sets as rounds land; the last wave to finish a tile reduces it in the
// fast-mode order of mfma_gemv.hpp.  Waiting waves sleep and the copy wave wakes them when
// it posts, so they take no issue slots from the computing ones.
// Tiles come in groups whose results combine:
//   gate/up: group (slot s, 8-row tile it of I) = the gate tile and the up tile of s's expert
//            against x; the second of the two to finish writes h[s][it*8 .. +8];
//   down:    group = 8-row tile it of H, one tile per slot, slot s against h[s]; the last slot
//            to finish combines  facc = f32(facc + f32(w_s * bf16(y_s)))  in slot order (w = 1
//            for the shared slot), y = bf16(facc) (tools/glm_model_q4k_ref.py:797-809), plus
//            the optional residual y = bf16(resid + y).
// Gate/up computes its routing decision in every workgroup from the router logits
// (route.hpp; workgroup 0 publishes it for the down leg and the caller); the down leg reads it.
#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"
#include "mfma_gemv.hpp"
#include "persist.hpp"
#include "route.hpp"

namespace aipu {

using namespace mg;
using namespace pst;

namespace {

constexpr int kMR = 8;         // rows per tile
constexpr int kMaxSlots = 9;   // topk routed + the shared slot
constexpr int kMaxNp = 16;     // block pairs per row (K <= 8192)
constexpr int kNcw = 12;       // compute waves (+ 1 copy wave)

struct TileSrc {
    const uint8_t* base;   // row 0 of the tile
    int nvalid;            // rows that exist (the rest read as zero)
    int act;               // activation vector
};

// ---------------------------------------------------------------- the two problems
struct PGateUp {
    const uint8_t *G, *U, *shG, *shU;
    int topk, nslots, E, itiles, ngroups;
    int64_t rb, ebytes, I;
    const uint16_t* X;
    uint16_t* h;
    MoeRoute route;
    static constexpr int kNA = 1;                                   // one activation vector (x)
    static constexpr int kStageBytes = kMaxNp * (int)kStage;        // its pairs
    __device__ int per_group() const { return 2; }
    __device__ TileSrc src(int wg, int grid, int t, const int32_t* eid) const {
        const int gi = wg + (t >> 1) * grid, s = gi / itiles, it = gi - s * itiles, part = t & 1;
        const uint8_t* base = s < topk ? (part ? U : G) + (int64_t)eid[s] * ebytes : (part ? shU : shG);
        return TileSrc{base + (int64_t)it * kMR * rb, kMR, 0};
    }
    __device__ const uint16_t* act(int) const { return X; }
    // lanes 0..7 (row r) of the wave that finished group g's second tile
    __device__ void combine(int wg, int grid, int g, const float* stash, int r) const {
        const int gi = wg + g * grid, s = gi / itiles, it = gi - s * itiles;
        const uint32_t gb = bf16_rne(stash[(2 * g) * kMR + r]), ub = bf16_rne(stash[(2 * g + 1) * kMR + r]);
        h[(int64_t)s * I + (int64_t)it * kMR + r] = (uint16_t)bf16_rne(bf16_to_f32(glm_silu_bf16(gb)) * bf16_to_f32(ub));
    }
};

struct PDown {
    const uint8_t *D, *shD;
    int topk, nslots, E, ngroups;
    int64_t rb, ebytes, H, I;
    const uint16_t* h;
    uint16_t* y;
    const uint16_t* resid;
    const int32_t* sel;
    const uint16_t* selw;
    static constexpr int kNA = kMaxSlots;                            // h[s], one per slot
    static constexpr int kStageBytes = kMaxSlots * 4 * (int)kStage;  // I <= 2048: 4 pairs each
    __device__ int per_group() const { return nslots; }
    __device__ TileSrc src(int wg, int grid, int t, const int32_t* eid) const {
        const int g = t / nslots, s = t - g * nslots, it = wg + g * grid;
        const uint8_t* base = s < topk ? D + (int64_t)eid[s] * ebytes : shD;
        const int64_t r0 = (int64_t)it * kMR, nv = H - r0;
        return TileSrc{base + r0 * rb, (int)(nv < kMR ? nv : kMR), s};
    }
    __device__ const uint16_t* act(int a) const { return h + (int64_t)a * I; }
    __device__ void combine(int wg, int grid, int g, const float* stash, int r, const uint16_t* w) const {
        const int64_t d = (int64_t)(wg + g * grid) * kMR + r;
        if (d >= H) return;
        float facc = 0.f;
        for (int s = 0; s < nslots; ++s) {
            const float yb = bf16_to_f32(bf16_rne(stash[(g * nslots + s) * kMR + r]));
            const float p = s < topk ? bf16_to_f32(w[s]) * yb : yb;
            facc = facc + p;
        }
        uint32_t yb = bf16_rne(facc);
        if (resid) yb = bf16_rne(bf16_to_f32(resid[d]) + bf16_to_f32(yb));
        y[d] = (uint16_t)yb;
    }
};

// ---------------------------------------------------------------- the kernel
// A tile (8 rows x rb bytes, rb a multiple of 128) sits in LDS chunk-major: the 16-byte chunk c
// of row r at 16 * (8c + r), so byte o (16-aligned) of row r is at 8o + 16r.  One direct-to-LDS
// load (64 lanes x 16 B, contiguous in LDS) then carries 128 bytes of each of the 8 rows, and
// the 8 rows' reads of one chunk are 128 contiguous bytes.  A round is kLoads such loads
// (1152 bytes of each row); a tile is R rounds.
constexpr int kLoads = 9;
constexpr uint32_t kRoundRow = 128u * kLoads;   // bytes of a row per round

__device__ __forceinline__ const uint8_t* uniform_ptr(const uint8_t* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint8_t*)(((uint64_t)hi << 32) | lo);
}

// R rounds per tile (row bytes rb = R * kRoundRow, so K = 2048 R: nsb = 8R blocks, np = 4R
// block pairs), TT tiles per workgroup at most (groups of per_group() tiles), NB tile buffers,
// Q rounds in flight.
template <class P, int R, int TT, int NB, int Q>
__global__ __launch_bounds__(64 * (kNcw + 1)) void k_moe_p(P pp) {
    constexpr int nsb = 8 * R, np = 4 * R;
    constexpr uint32_t rb = R * kRoundRow;
    static_assert(np <= kMaxNp, "block pairs per row");
    // a buffer is reused once its previous tile is reduced, and that tile's last round must be
    // posted by then: Q - 1 rounds stay unposted, so Q <= (NB - 1) * R + 1
    static_assert(Q >= 1 && Q <= (NB - 1) * R + 1, "rounds in flight vs buffer reuse");
    static_assert(kLoads * (Q - 1) <= 63, "rounds in flight within vmcnt");
    extern __shared__ __align__(16) uint8_t s_tile[];                 // direct-to-LDS targets only
    __shared__ __align__(16) uint8_t s_stage[P::kStageBytes];
    __shared__ __align__(16) float s_red[NB * kMR * kMaxNp];
    __shared__ float s_stash[TT * kMR];
    __shared__ uint32_t s_cnt[TT * R], s_done[TT], s_freed[TT], s_gdone[TT], s_staged;
    __shared__ int32_t s_eid[kMaxSlots];
    __shared__ uint16_t s_w[kMaxSlots];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x, G = gridDim.x;
    const int npg = pp.per_group();
    const int T = (pp.ngroups - wg + G - 1) / G * npg;                // this workgroup's tiles
    constexpr uint32_t TB = kMR * rb;
    for (int i = tid; i < TT * R; i += blockDim.x) s_cnt[i] = 0u;
    if (tid < TT) {
        s_done[tid] = 0u;
        s_freed[tid] = 0u;
        s_gdone[tid] = 0u;
    }
    if (tid == 0) s_staged = 0u;

    // ---- the routing decision (expert id per slot) before any weight address is known
    if constexpr (P::kNA == 1) {
        __shared__ __align__(16) uint32_t r_keys[kRouteMaxE];
        __shared__ uint32_t r_win[kRouteMaxTopk];
        __shared__ int32_t r_sel[kRouteMaxTopk];
        __shared__ uint16_t r_selw[kRouteMaxTopk];
        if (pp.route.logits) {
            route_workgroup(pp.route.logits, pp.E, pp.topk, pp.route.scale_bits, r_keys, r_win, r_sel, r_selw, wg == 0);
            if (tid < pp.topk) {
                const int e = (int)(0xFFFFu - (r_win[tid] & 0xFFFFu));
                s_eid[tid] = e < 0 ? 0 : (e >= pp.E ? pp.E - 1 : e);
                if (wg == 0) {
                    pp.route.sel_pub[tid] = r_sel[tid];
                    pp.route.selw_pub[tid] = r_selw[tid];
                    if (pp.route.sel_api) pp.route.sel_api[tid] = r_sel[tid];
                    if (pp.route.selw_api) pp.route.selw_api[tid] = r_selw[tid];
                }
            }
        } else if (tid < pp.topk) {
            const int e = pp.route.sel[tid];
            s_eid[tid] = e < 0 ? 0 : (e >= pp.E ? pp.E - 1 : e);
        }
    } else {
        if (tid < pp.topk) {
            const int e = pp.sel[tid];
            s_eid[tid] = e < 0 ? 0 : (e >= pp.E ? pp.E - 1 : e);
            s_w[tid] = pp.selw[tid];
        }
    }
    if (tid == pp.topk && pp.topk < kMaxSlots) s_eid[tid] = 0;   // the shared slot (unused id)
    __syncthreads();   // routing, counters

    const int n = lane & 15, g = lane >> 4, h = n >> 3, r = n & 7;
    if (w == kNcw) {
        // ---- copy wave: round u = t * R + k, Q in flight, each posted once its loads landed.
        // A runtime loop with one fixed wait keeps this wave's code small, so the compute
        // waves' loop stays in the instruction cache.
        // The wave issues at raised priority: its loads must not queue behind the compute
        // waves' instructions.
        __builtin_amdgcn_s_setprio(3);
        uint32_t cnt0 = lds_addr(s_cnt);
        asm volatile("" : "+v"(cnt0));   // a runtime base (see lds_post)
        const uint32_t loff = (uint32_t)(lane & 7) * rb + 16u * (uint32_t)(lane >> 3);   // lane's bytes in a load
        const int U = T * R;
        int posted = 0;
        for (int u = 0; u < U; ++u) {
            const int t = u / R, k = u - t * R;
            if (k == 0 && t >= NB) spin_ge(&s_freed[t - NB], 1u);
            const TileSrc sr = pp.src(wg, G, t, s_eid);
            const int nvalid = __builtin_amdgcn_readfirstlane(sr.nvalid);
            const __amdgpu_buffer_rsrc_t wr = buf_rsrc(uniform_ptr(sr.base), (uint32_t)nvalid * rb);
            uint8_t* dst = s_tile + (uint32_t)(t % NB) * TB + 1024u * kLoads * (uint32_t)k;
            const uint32_t off = loff + kRoundRow * (uint32_t)k;
#pragma unroll
            for (int j = 0; j < kLoads; ++j) lds_dma16<kNT>(wr, dst + 1024u * j, off + 128u * j);
            if (u >= Q - 1) {
                __builtin_amdgcn_s_waitcnt(wait_vm(kLoads * (Q - 1)));
                lds_post_wake(cnt0 + 4u * (uint32_t)posted);
                ++posted;
            }
        }
        // the last rounds: the oldest of `left` unposted rounds has landed once kLoads * (left - 1)
        // loads remain
        const int left = U - posted;
        static_for<0, Q - 1>([&](auto sI) {
            constexpr int j = Q - 2 - decltype(sI)::value;
            if (j < left) {
                __builtin_amdgcn_s_waitcnt(wait_vm(kLoads * j));
                lds_post_wake(cnt0 + 4u * (uint32_t)posted);
                ++posted;
            }
        });
        return;
    }

    // ---- compute waves: stage the activations
    u32x4_t A[8];
    float2 as = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) A[i] = u32x4_t{0u, 0u, 0u, 0u};
    if constexpr (P::kNA == 1) {
        // wave w owns pair w (kNcw == np): its operands stay in registers
        if (w < np) {
            const __amdgpu_buffer_rsrc_t xr = buf_rsrc(pp.act(0), (uint32_t)nsb * 512u);
            const uint4 xv = buf_load16(xr, (uint32_t)w * 1024u + 16u * (uint32_t)lane);
            uint8_t* st = s_stage + (uint32_t)w * kStage;
            stage_pair(xv, st, lane);
            read_pair_operands(A, as, lds_addr(st), g, n);
        }
    } else {
        // job j = (activation a, pair p), a < nslots: wave w stages jobs w, w + kNcw, ...
        constexpr int kJobs = (kMaxSlots * 4 + kNcw - 1) / kNcw;
        const int njobs = pp.nslots * np;
        uint4 xv[kJobs];
#pragma unroll
        for (int i = 0; i < kJobs; ++i) {
            const int j = w + kNcw * i, a = j / np, p = j - a * np;
            const __amdgpu_buffer_rsrc_t xr = buf_rsrc(pp.act(j < njobs ? a : 0), (uint32_t)nsb * 512u);
            xv[i] = buf_load16(xr, j < njobs ? (uint32_t)p * 1024u + 16u * (uint32_t)lane : kOOB);
        }
#pragma unroll
        for (int i = 0; i < kJobs; ++i) {
            const int j = w + kNcw * i;
            if (j < njobs) stage_pair(xv[i], s_stage + (uint32_t)j * kStage, lane);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        lds_post(&s_staged);
        spin_ge(&s_staged, (uint32_t)kNcw);
    }

    // ---- the sets: (tile t, pair p) is wave (t * np + p) % kNcw's (with one activation,
    // kNcw == np, so that is the pair's owner)
    const HdrSel hs = hdr_sel(g);
    const CodeK ck = code_k();
    int seen = -1;
    // this wave's sets in order: flat index t * np + p = w, w + kNcw, ...
    for (int t = w / np, p = w % np; t < T; t += (p + kNcw) / np, p = (p + kNcw) % np) {
        {
            const uint32_t pend = 288u * (uint32_t)p + 287u < rb ? 288u * (uint32_t)p + 287u : rb - 1u;
            const int u = t * R + (int)(pend / kRoundRow);
            // header of block 2p + h at byte 144 (2p + h), its qs for K-group g 32 bytes at 16 + 32g
            const uint32_t oh = 144u * (2u * (uint32_t)p + (uint32_t)h);
            const uint32_t tl = lds_addr(s_tile) + (uint32_t)(t % NB) * TB + 16u * (uint32_t)r;
            const uint32_t ah = tl + 8u * oh, aq = tl + 8u * (oh + 16u + 32u * (uint32_t)g);
            u32x4_t hv, q0, q1;
            uint32_t cv;
            asm volatile(
                "ds_read_b32 %3, %6\n\t"
                "ds_read_b128 %0, %4\n\t"
                "ds_read_b128 %1, %5\n\t"
                "ds_read_b128 %2, %5 offset:128\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(hv), "=&v"(q0), "=&v"(q1), "=&v"(cv)
                : "v"(ah), "v"(aq), "v"(lds_addr(&s_cnt[u]))
                : "memory");
            if (seen < u && __builtin_amdgcn_readfirstlane(cv) < 1u) {
                wait_woken(&s_cnt[u], 1u);
                asm volatile(
                    "ds_read_b128 %0, %3\n\t"
                    "ds_read_b128 %1, %4\n\t"
                    "ds_read_b128 %2, %4 offset:128\n\t"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(hv), "=&v"(q0), "=&v"(q1)
                    : "v"(ah), "v"(aq)
                    : "memory");
            }
            seen = seen < u ? u : seen;
            if constexpr (P::kNA != 1) {
                const int a = pp.src(wg, G, t, s_eid).act;
                read_pair_operands(A, as, lds_addr(s_stage) + (uint32_t)(a * np + p) * kStage, g, n);
            }
            const float bt = pair_block_term(A, as, hv, q0, q1, hs, ck, h);
            const float b1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(bt), 0x108, 0xF, 0xF, false));
            const float ps = bt + (2 * p + 1 < nsb ? b1 : 0.0f);
            float* rt = s_red + (t % NB) * (kMR * kMaxNp);
            if (lane < kMR) rt[lane * kMaxNp + p] = ps;
            // (a wave's DS operations execute in order: its pair sums land before its count)
            if (lds_add_rtn(&s_done[t]) != (uint32_t)np - 1u) continue;
            // the tile's last pair: its 8 sums, then the group's combine if this was its last tile
            const float v = tile_tree(rt, kMaxNp, np, lane);
            if ((lane & 7) == 0) s_stash[t * kMR + (lane >> 3)] = v;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // rt read, stash written
            lds_post(&s_freed[t]);
            const int grp = t / npg;
            if (lds_add_rtn(&s_gdone[grp]) != (uint32_t)npg - 1u) continue;
            if (lane < kMR) {
                if constexpr (P::kNA == 1) pp.combine(wg, G, grp, s_stash, lane);
                else pp.combine(wg, G, grp, s_stash, lane, s_w);
            }
        }
    }
}

template <class P, int R, int TT, int NB, int Q>
hipError_t run_p(const P& pp, int64_t K, int G, hipStream_t st) {
    if (row_bytes(T_Q4_K, K) != (int64_t)R * kRoundRow) return hipErrorInvalidValue;
    const size_t lds = (size_t)NB * kMR * R * kRoundRow;
    hipLaunchKernelGGL((k_moe_p<P, R, TT, NB, Q>), dim3(G), dim3(64 * (kNcw + 1)), lds, st, pp);
    return hipGetLastError();
}

// tile buffers and rounds in flight per leg (gate/up: 3 rounds per tile, down: 1)
constexpr int kGuNB = 4, kGuQ = 5, kDnNB = 8, kDnQ = 5;

int cus() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, v = 0;
        n = hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                ? v : 256;
    }
    return n;
}

// groups per workgroup of each leg when every CU holds one workgroup
int gateup_groups_per_wg(int nslots, int64_t I) { return (int)((nslots * (I / kMR) + cus() - 1) / cus()); }
int down_groups_per_wg(int64_t H) { return (int)(((H + kMR - 1) / kMR + cus() - 1) / cus()); }

}  // namespace

// The persistent legs serve the config-2 shape class: hidden 6144 (12 block pairs, one per
// compute wave), intermediate 2048, 8 routed slots with or without the shared slot, at most
// one routing key per thread of a workgroup, and a CU count that gives the instantiated
// tiles per workgroup (8 or 9 gate/up groups, 3 down groups: 256 CUs).
bool moe_persist_supported(int nslots, int topk, int64_t E, int64_t H, int64_t I) {
    return H == 6144 && I == 2048 && topk == 8 && (nslots == 8 || nslots == 9) && E >= topk &&
           E <= kRouteMaxE && E <= 64 * (kNcw + 1) && gateup_groups_per_wg(nslots, I) == nslots &&
           down_groups_per_wg(H) == 3;
}

hipError_t launch_moe_gateup_persist(const uint8_t* G, const uint8_t* U, const uint8_t* shG, const uint8_t* shU,
                                     const MoeRoute& route, int topk, int nslots, int64_t E, int64_t H, int64_t I,
                                     const uint16_t* x, uint16_t* h, hipStream_t st) {
    if (!moe_persist_supported(nslots, topk, E, H, I)) return hipErrorInvalidValue;
    const int64_t rb = row_bytes(T_Q4_K, H);
    const int itiles = (int)(I / kMR), ngroups = nslots * itiles;
    const int ng = gateup_groups_per_wg(nslots, I);
    const int Gn = (ngroups + ng - 1) / ng;
    const PGateUp pp{G, U, shG, shU, topk, nslots, (int)E, itiles, ngroups, rb, rb * I, I, x, h, route};
    if (ng == 8) return run_p<PGateUp, 3, 16, kGuNB, kGuQ>(pp, H, Gn, st);
    if (ng == 9) return run_p<PGateUp, 3, 18, kGuNB, kGuQ>(pp, H, Gn, st);
    return hipErrorInvalidValue;
}

hipError_t launch_moe_down_persist(const uint8_t* D, const uint8_t* shD, const int32_t* sel, const uint16_t* selw,
                                   int topk, int nslots, int64_t E, int64_t H, int64_t I, const uint16_t* h,
                                   uint16_t* y, const uint16_t* resid, hipStream_t st) {
    if (!moe_persist_supported(nslots, topk, E, H, I)) return hipErrorInvalidValue;
    const int64_t rb = row_bytes(T_Q4_K, I);
    const int ngroups = (int)((H + kMR - 1) / kMR);
    const int ng = down_groups_per_wg(H);
    const int Gn = (ngroups + ng - 1) / ng;
    const PDown pp{D, shD, topk, nslots, (int)E, ngroups, rb, rb * H, H, I, h, y, resid, sel, selw};
    if (ng == 3 && nslots == 8) return run_p<PDown, 1, 24, kDnNB, kDnQ>(pp, I, Gn, st);
    if (ng == 3 && nslots == 9) return run_p<PDown, 1, 27, kDnNB, kDnQ>(pp, I, Gn, st);
    return hipErrorInvalidValue;
}

}  // namespace aipu
