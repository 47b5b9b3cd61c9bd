// Persistent matrix-core MoE expert legs for the single-row decode step (tolerance mode):
// topk <= 8 routed slots and an optional shared expert as the last slot, H = 2048 R (R <= 3),
// I = 2048.
// Mirrors the expert half of decoder_block (tools/glm_model_q4k_ref.py:797-809) with
// swiglu_expert (:702-708); the routing decision is route.hpp's (:663-699).
//
// Both legs run one workgroup per CU over a list of jobs, with the memory plan of the
// persistent multi-row GEMV: the copy waves (12, and 13 in the gate/up leg) take turns copying
// rounds of 8 rows x 1152 B (4 block pairs, nine direct-to-LDS loads of 64 lanes x 16 B,
// chunk-major: 16-B chunk c of row r at 16 (8c + r)) into a ring of NS LDS slots, post each
// round to an LDS counter once it has landed, and refill a slot once the four sets that read
// it hold their weights in registers.  Compute
// wave w = 4 gamma + p takes block pair p (a set: 8 rows x 2 blocks, one pass of 8 MFMAs) of
// the rounds of group gamma; the last set of a job reduces the job.
//
// Gate/up (k_moe_gu_p): job = (slot s, rows i0 .. i0+7 of I); round q = 0 .. 2R-1 holds K
// segment k = q % R of the gate rows (q < R) or the up rows (q >= R) of expert sel[s] (the
// shared expert's for the last slot when there is one).  Group
// gamma takes the rounds with k = gamma, so wave 4k + p always meets block pair 4k + p of x
// and keeps that pair's operands in registers for the whole kernel.  Reduction per row: the
// 4R pair sums in a fixed order, then h = bf16(silu(bf16(g)) * bf16(u)).  Every workgroup
// routes from the router logits itself before its first weight copy; workgroup 0 publishes
// the decision for the down leg and the caller.  Once a copy wave has issued its own rounds it
// loads the first kDnPrefetch rounds of the down leg's workgroup wg (slots 0, 1, ... of output
// rows 8 wg ..) into a scratch kilobyte of LDS and waits for them, so that they sit in the
// caches when the down leg starts (measured 0.4-0.5 us off the step).
//
// Down (k_moe_down_p): job = output rows d0 .. d0+7; round q = slot q (8 rows x 1152 B of
// expert sel[q] or the shared expert, all I = 2048 weights of the rows); group gamma takes the slots q = gamma
// mod 3 and stages those slots' activation pairs h[q] in LDS.  Reduction per row: per slot
// y_s = (s0 + s1) + (s2 + s3) over its pair sums, then the slot-ordered combine
//     facc = f32(facc + f32(w_s * bf16(y_s)))   (tools/glm_model_q4k_ref.py:799-809),
// the shared slot last with w = 1; y = bf16(facc), or bf16(resid + bf16(facc)) with the
// decoder block's residual.
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

constexpr int kJR = 8;                        // rows per job tile
constexpr int kLoads = 9;                     // direct-to-LDS loads per round
constexpr uint32_t kRoundRow = 128u * kLoads; // bytes of a row per round (4 block pairs)
constexpr uint32_t kSlot = kJR * kRoundRow;   // bytes of a round
constexpr int kReaders = 4;                   // sets that read a round
constexpr int kNCW = 12;                      // compute waves
constexpr int kGroups = 3;                    // compute wave groups of 4
constexpr int kMaxJobs = 9;                   // jobs per workgroup
constexpr int kMaxRouted = 8;                 // routed slots
constexpr int kMaxSlots = kMaxRouted + 1;     // and the shared expert
constexpr int kMaxRJ = kMaxSlots;             // rounds per job (down: one per slot; gate/up: 2R <= 6)
constexpr int kRedJob = kMaxSlots * kJR * 4;  // pair sums per job (floats; gate/up uses 16 x 12)
constexpr int kGuNp = 12;                     // pair-sum stride of a gate/up row (4R <= 12)
constexpr int kDnPrefetch = 7;                // down-leg rounds per workgroup the gate/up leg prefetches (its first Q)

// Nine loads of round k of 8 rows (row stride rb) at `base` into the LDS slot `dst`.
template <uint32_t POL>
__device__ __forceinline__ void issue_round(const uint8_t* base, int nvalid, uint32_t rb, uint32_t k, uint8_t* dst,
                                            int lane) {
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(base, (uint32_t)nvalid * rb);
    const uint32_t off = (uint32_t)(lane & 7) * rb + 16u * (uint32_t)(lane >> 3) + kRoundRow * k;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) lds_dma16<POL>(wr, dst + 1024u * j, off + 128u * j);
}

// The weights of one set (block pair pp of the round in slot address sl; lane 16g + n reads
// the header and qs chunk g of block 2pp + h, row r) and the round counter, in one LDS batch:
// a posted counter proves that the weights read after it (in DS order) had landed;
// otherwise wait for the post and read again.
__device__ __forceinline__ void set_weights(uint32_t sl, uint32_t cnt, int pp, int h, int r, int g, bool known,
                                            u32x4_t& hv, u32x4_t& q0, u32x4_t& q1) {
    const uint32_t oh = 288u * (uint32_t)pp + 144u * (uint32_t)h;
    const uint32_t tl = sl + 16u * (uint32_t)r;
    const uint32_t ah = tl + 8u * oh, aq = tl + 8u * (oh + 16u + 32u * (uint32_t)g);
    uint32_t cv;
    asm volatile(
        "ds_read_b32 %3, %6\n\t"
        "ds_read_b128 %0, %4\n\t"
        "ds_read_b128 %1, %5\n\t"
        "ds_read_b128 %2, %5 offset:128\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(hv), "=&v"(q0), "=&v"(q1), "=&v"(cv)
        : "v"(ah), "v"(aq), "v"(cnt)
        : "memory");
    if (!known && (uint32_t)__builtin_amdgcn_readfirstlane(cv) < 1u) {
        for (uint32_t it = 0;; ++it) {
            uint32_t c;
            asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(c) : "v"(cnt) : "memory");
            if ((uint32_t)__builtin_amdgcn_readfirstlane(c) >= 1u) break;
            if (it == (1u << 22)) {   // give up (recorded), as spin_ge does
                wait_gave_up();
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        asm volatile(
            "ds_read_b128 %0, %3\n\t"
            "ds_read_b128 %1, %4\n\t"
            "ds_read_b128 %2, %4 offset:128\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(hv), "=&v"(q0), "=&v"(q1)
            : "v"(ah), "v"(aq)
            : "memory");
    }
}

// The block-diagonal operands of a staged pair (diagonal lanes 16g + 4g + h, h < 2; every
// other lane keeps its zeros) and this lane's sub-block sums.
__device__ __forceinline__ void pair_operands(uint32_t st, int g, int n, int h, u32x4_t (&A)[8], float2& as) {
    const uint32_t aa = st + 32u * (uint32_t)g + 16u * (uint32_t)((n - 4 * g) & 1);
    uint64_t saved;
    asm volatile(
        "s_mov_b64 %[sv], exec\n\t"
        "s_and_b64 exec, exec, %[mask]\n\t"
        "ds_read_b128 %[a0], %[aa]\n\t"
        "ds_read_b128 %[a1], %[aa] offset:144\n\t"
        "ds_read_b128 %[a2], %[aa] offset:288\n\t"
        "ds_read_b128 %[a3], %[aa] offset:432\n\t"
        "ds_read_b128 %[a4], %[aa] offset:576\n\t"
        "ds_read_b128 %[a5], %[aa] offset:720\n\t"
        "ds_read_b128 %[a6], %[aa] offset:864\n\t"
        "ds_read_b128 %[a7], %[aa] offset:1008\n\t"
        "s_mov_b64 exec, %[sv]\n\t"
        "ds_read_b64 %[as], %[sa]\n\t"
        "s_waitcnt lgkmcnt(0)"
        : [a0] "+v"(A[0]), [a1] "+v"(A[1]), [a2] "+v"(A[2]), [a3] "+v"(A[3]), [a4] "+v"(A[4]), [a5] "+v"(A[5]),
          [a6] "+v"(A[6]), [a7] "+v"(A[7]), [as] "=&v"(as), [sv] "=&s"(saved)
        : [aa] "v"(aa), [mask] "s"(diag_mask(2)), [sa] "v"(st + kStgSums + 8u * (uint32_t)(g * 2 + h))
        : "memory", "scc");   // s_and_b64 writes SCC
}

// One set: the pair sum (block 2pp + block 2pp + 1) of tile row r on lanes 0 .. 7.
__device__ __forceinline__ float set_sum(const u32x4_t (&A)[8], float2 as, const u32x4_t& hv, const u32x4_t& q0,
                                         const u32x4_t& q1, const HdrSel& hs, const CodeK& ck, int h) {
    f32x4_t dlo, dhi;
    dlo[0] = dlo[1] = -kCodeBiasF * as.x;
    dhi[0] = dhi[1] = -kCodeBiasF * as.y;
    dlo[2] = dlo[3] = dhi[2] = dhi[3] = 0.f;
    const uint32_t qd[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        dlo = mfma(A[tt], codes_lo(qd[2 * tt], qd[2 * tt + 1], ck), dlo);
        dhi = mfma(A[4 + tt], codes_hi(qd[2 * tt], qd[2 * tt + 1], ck), dhi);
    }
    const Hdr H = hdr_decode(make_uint4(hv.x, hv.y, hv.z, hv.w), hs);
    const float bt = block_sum(block_term(H, h ? dlo[1] : dlo[0], h ? dhi[1] : dhi[0], as.x, as.y));
    const float b1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(bt), 0x108, 0xF, 0xF, false));
    return bt + b1;
}

// ---------------------------------------------- fp16 high-nibble operands (gate/up leg)
// The gate/up leg builds the high-nibble codes as fp16 1024 + 16 q = (x & 0x00F0) | 0x6400, which
// needs no shift (the low-nibble codes stay bf16 128 + q). Their MFMAs take the pair's
// activations as fp16 scaled by 2^-e, e putting the pair's largest magnitude in [2^14, 2^15):
// every bf16 value down to 2^-24 of it converts exactly, and a' (1024 + 16 q) is exact in fp32.
// Seeded with -1024 * 2^-e * sum a, the chain ends at 16 * 2^-e * sum a q, which 2^(e - 4) scales
// back exactly. This leg's order is its own (compared with exact arithmetic within the MoE bound).
struct CodeKH {
    uint32_t mask;   // wave-uniform (SGPR)
    uint32_t bias;   // VGPR
};

__device__ __forceinline__ CodeKH code_kh() {
    CodeKH k;
    k.mask = 0x00F000F0u;
    k.bias = 0x64006400u;   // fp16 1024.0 in both halves
    asm volatile("" : "+s"(k.mask));
    asm volatile("" : "+v"(k.bias));
    return k;
}

// The high-nibble B operands of codes_hi in the same element places, as fp16 1024 + 16 q.
__device__ __forceinline__ u32x4_t codes_hi16(uint32_t x0, uint32_t x1, const CodeKH& k) {
    return u32x4_t{(x0 & k.mask) | k.bias, ((x0 >> 8) & k.mask) | k.bias, (x1 & k.mask) | k.bias,
                   ((x1 >> 8) & k.mask) | k.bias};
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4_t mfma16(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                  0, 0);
}

// The exponent e of a pair (64 lanes of 8 bf16) for its fp16 operands; 0 for an all-zero pair or
// one holding inf / nan.
__device__ __forceinline__ int pair_exponent(const uint4& xv) {
    const uint32_t v[4] = {xv.x, xv.y, xv.z, xv.w};
    uint32_t mx = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) mx = max(mx, max(v[k] & 0x7FFFu, (v[k] >> 16) & 0x7FFFu));
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, s, 64));
    if (mx == 0 || mx >= 0x7F80u) return 0;
    int ex;
    (void)frexpf(bf16_to_f32(mx), &ex);   // max = f * 2^ex, f in [0.5, 1)
    return ex - 15;
}

// Two bf16 (one dword) times 2^-e as an fp16 pair, round to nearest even.
__device__ __forceinline__ uint32_t f16_pair_scaled(uint32_t w, int e) {
    const float lo = __builtin_ldexpf(__uint_as_float(w << 16), -e);
    const float hi = __builtin_ldexpf(__uint_as_float(w & 0xFFFF0000u), -e);
    return (uint32_t)__half_as_ushort(__float2half_rn(lo)) | ((uint32_t)__half_as_ushort(__float2half_rn(hi)) << 16);
}

// x pair pr into registers as x_operands does, the high-nibble operands (MFMAs t >= 4) as fp16
// scaled by 2^-e; the sub-block sums stay those of the bf16 values.
__device__ __forceinline__ void x_operands16(const uint4& xv, uint8_t* st, int lane, int e, u32x4_t (&A)[8],
                                             float2& as) {
    const int n = lane & 15, g = lane >> 4, h = n >> 3;
    stage_pair(xv, st, lane);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if ((lane & 7) >= 4) {   // chunk t = lane & 7 of the pair: rewrite its entry in fp16
        const uint4 hv = make_uint4(f16_pair_scaled(xv.x, e), f16_pair_scaled(xv.y, e), f16_pair_scaled(xv.z, e),
                                    f16_pair_scaled(xv.w, e));
        const int L = lane, hh = L >> 5, gg = (L >> 3) & 3, t = L & 7;
        *(u32x4_t*)(st + 16u * (uint32_t)(9 * t + 2 * gg + hh)) = act_perm(hv);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) A[i] = u32x4_t{0u, 0u, 0u, 0u};
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    pair_operands(lds_addr(st), g, n, h, A, as);
}

// set_sum with the high-nibble chain on fp16 operands: seeded with seed_hi = -1024 * 2^-e * as.y,
// its sum scaled by hscale = 2^(e - 4) before the block term.
__device__ __forceinline__ float set_sum16(const u32x4_t (&A)[8], float2 as, float seed_hi, float hscale,
                                           const u32x4_t& hv, const u32x4_t& q0, const u32x4_t& q1, const HdrSel& hs,
                                           const CodeK& ck, const CodeKH& kh, int h) {
    f32x4_t dlo, dhi;
    dlo[0] = dlo[1] = -kCodeBiasF * as.x;
    dhi[0] = dhi[1] = seed_hi;
    dlo[2] = dlo[3] = dhi[2] = dhi[3] = 0.f;
    const uint32_t qd[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        dlo = mfma(A[tt], codes_lo(qd[2 * tt], qd[2 * tt + 1], ck), dlo);
        dhi = mfma16(A[4 + tt], codes_hi16(qd[2 * tt], qd[2 * tt + 1], kh), dhi);
    }
    const Hdr H = hdr_decode(make_uint4(hv.x, hv.y, hv.z, hv.w), hs);
    const float shi = (h ? dhi[1] : dhi[0]) * hscale;
    const float bt = block_sum(block_term(H, h ? dlo[1] : dlo[0], shi, as.x, as.y));
    const float b1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(bt), 0x108, 0xF, 0xF, false));
    return bt + b1;
}

// ------------------------------------------------------------------ job loops
// LDS of a workgroup's ring: slots, per-round landed / read counters, per-job set counters,
// per-job pair sums.
struct Ring {
    uint8_t* slots;
    uint32_t *cnt, *read, *done;
    float* red;
};

// Copy-wave cursor over the gate/up rounds: round q (0 .. 2R-1) of the job of slot js and row
// group ji (rows 8 ji .. 8 ji + 7 of I); jobs wg, wg + G, ... in order.
struct GuCursor {
    int q, js, ji;
    __device__ void start(int q0, int wg, int it8, int RJ, int G) {
        q = q0;
        js = wg / it8;
        ji = wg - js * it8;
        advance(0, it8, RJ, G);
    }
    __device__ void advance(int by, int it8, int RJ, int G) {
        q += by;
        while (q >= RJ) {
            q -= RJ;
            ji += G;
            while (ji >= it8) {
                ji -= it8;
                ++js;
            }
        }
    }
};
// Expert matrices of one leg: the routed stack (expert e at e * ebytes) and the shared expert
// (slot topk, when there is one).
struct Stack {
    const uint8_t* base;
    const uint8_t* shared;
    int64_t ebytes;
    __device__ const uint8_t* slot(int ev, int s, int topk) const {
        return s < topk ? base + (int64_t)__builtin_amdgcn_readlane(ev, s) * ebytes : shared;
    }
};

template <int R, uint32_t POL>
__device__ __forceinline__ void gu_issue(const GuCursor& cu, int ev, const Stack& Gs, const Stack& Us, int topk,
                                         uint8_t* dst, int lane) {
    constexpr uint32_t rb = R * kRoundRow;
    const int half = cu.q >= R ? 1 : 0, k = cu.q - half * R;
    issue_round<POL>((half ? Us : Gs).slot(ev, cu.js, topk) + (int64_t)cu.ji * kJR * rb, kJR, rb, (uint32_t)k, dst,
                     lane);
}

// Copy-wave cursor over the down rounds: slot q of the job of output rows d0 .. d0 + 7.
struct DnCursor {
    int q;
    int64_t d0;
    __device__ void start(int i, int S, int wg, int G) {   // i-th down round of the workgroup
        q = i % S;
        d0 = (int64_t)(wg + (i / S) * G) * kJR;
    }
    __device__ void advance(int by, int S, int G) {
        q += by;
        while (q >= S) {
            q -= S;
            d0 += (int64_t)G * kJR;
        }
    }
};
template <uint32_t POL>
__device__ __forceinline__ void dn_issue(const DnCursor& cu, int ev, const Stack& Ds, int topk, int64_t Hd,
                                         uint8_t* dst, int lane) {
    const int nvalid = (int)(Hd - cu.d0 < kJR ? Hd - cu.d0 : kJR);
    issue_round<POL>(Ds.slot(ev, cu.q, topk) + cu.d0 * (int64_t)kRoundRow, nvalid, kRoundRow, 0u, dst, lane);
}

// Lane s < topk: slot s's expert from the winners' keys.
__device__ __forceinline__ int slot_experts(const uint32_t* win, int topk, int E, int lane) {
    if (lane >= topk) return 0;
    const int e = (int)(0xFFFFu - (win[lane] & 0xFFFFu));
    return e < 0 ? 0 : (e >= E ? E - 1 : e);
}

// Gate/up jobs of compute wave (gam, p), which holds block pair pr = 4 gam + p of x in A / as:
// job t's rounds are u0 + 2R t + half R + gam; the job's last set forms its 8 h values.
template <int R, int NS>
__device__ __forceinline__ void gu_jobs(const Ring& rg, int T, int u0, int wg, int G, int it8, int I, int gam, int p,
                                        const u32x4_t (&A)[8], float2 as, float seed_hi, float hscale,
                                        const HdrSel& hs, const CodeK& ck, const CodeKH& kh, int& seen,
                                        uint16_t* __restrict__ Hout, int lane) {
    constexpr int RJ = 2 * R, np = 4 * R;
    const int n = lane & 15, g = lane >> 4, h = n >> 3, r = n & 7;
    const int pr = 4 * gam + p;
    for (int t = 0; t < T; ++t) {
        float* rt = rg.red + t * kRedJob;   // [gate rows 0..7, up rows 8..15][pair]
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int u = u0 + t * RJ + half * R + gam;
            u32x4_t hv, q0, q1;
            set_weights(lds_addr(rg.slots) + (uint32_t)(u % NS) * kSlot, lds_addr(&rg.cnt[u]), p, h, r, g, seen >= u,
                        hv, q0, q1);
            seen = seen < u ? u : seen;
            lds_post(&rg.read[u]);   // the weights are in registers: one reader fewer
            const float ps = set_sum16(A, as, seed_hi, hscale, hv, q0, q1, hs, ck, kh, h);
            if (lane < kJR) rt[(half * kJR + lane) * kGuNp + pr] = ps;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // pair sums written before the count
        if (lds_add_rtn(&rg.done[t]) != (uint32_t)np - 1u) continue;   // one post per wave and job
        // the job's last set: lane 4 * row + k (rows 0..7 gate, 8..15 up) sums pairs k, k + 4, ...
        const int row = lane >> 2, k = lane & 3;
        float v = rt[row * kGuNp + k];
#pragma unroll
        for (int jj = k + 4; jj < np; jj += 4) v += rt[row * kGuNp + jj];
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));   // xor 1
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));   // xor 2
        const float uvl = __shfl_xor(v, 32, 64);   // up row i sits 32 lanes above gate row i
        const int j = wg + t * G;
        const int s = j / it8, i0 = (j - s * it8) * kJR;
        if (lane < 32 && k == 0) {
            const uint32_t gb = bf16_rne(v), ub = bf16_rne(uvl);
            Hout[(int64_t)s * I + i0 + row] = (uint16_t)bf16_rne(bf16_to_f32(glm_silu_bf16(gb)) * bf16_to_f32(ub));
        }
    }
}

// Down jobs of compute wave (gam, p): slots q = gam, gam + 3, ... of job t are rounds
// u0 + S t + q, against staged pair 4q + p; the job's last set combines the slots.
template <int NS>
__device__ __forceinline__ void dn_jobs(const Ring& rg, int T, int u0, int S, int topk, int wg, int G, int64_t Hd,
                                        int gam, int p, uint32_t stage, const HdrSel& hs, const CodeK& ck, int& seen,
                                        const uint16_t* selw, uint16_t* __restrict__ Y,
                                        const uint16_t* __restrict__ resid, int lane) {
    const int n = lane & 15, g = lane >> 4, h = n >> 3, r = n & 7;
    u32x4_t A[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) A[i] = u32x4_t{0u, 0u, 0u, 0u};
    const int mine = gam < S ? (S - gam + kGroups - 1) / kGroups : 0;   // slots this wave takes
    for (int t = 0; t < T; ++t) {
        float* rt = rg.red + t * kRedJob;   // [slot][row][pair]
        for (int q = gam; q < S; q += kGroups) {
            const int u = u0 + t * S + q;
            u32x4_t hv, q0, q1;
            set_weights(lds_addr(rg.slots) + (uint32_t)(u % NS) * kSlot, lds_addr(&rg.cnt[u]), p, h, r, g, seen >= u,
                        hv, q0, q1);
            seen = seen < u ? u : seen;
            lds_post(&rg.read[u]);   // the weights are in registers: one reader fewer
            float2 as;
            pair_operands(stage + (uint32_t)(4 * q + p) * kStgBytes, g, n, h, A, as);
            const float ps = set_sum(A, as, hv, q0, q1, hs, ck, h);
            if (lane < kJR) rt[(q * kJR + lane) * 4 + p] = ps;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // pair sums written before the count
        // one post per set; the wave whose post completes the job's 4S sets reduces it
        uint32_t before = 0;
        for (int i = 0; i < mine; ++i) before = lds_add_rtn(&rg.done[t]);
        if (mine == 0 || before != (uint32_t)(4 * S) - 1u) continue;
        // the job's last set: lane 8 * row + slot (slots 0..7; a ninth slot, the shared expert
        // after eight routed ones, is formed by lane 8 * row itself); weight 1 for the shared slot
        const int row = lane >> 3, s = lane & 7;
        const auto slot_term = [&](int q) {
            const float* qp = rt + (q * kJR + row) * 4;
            const float yb = bf16_to_f32(bf16_rne((qp[0] + qp[1]) + (qp[2] + qp[3])));
            return q < topk ? bf16_to_f32(selw[q]) * yb : yb;
        };
        const float pw = s < S ? slot_term(s) : 0.f;
        float facc = 0.f;
        for (int s2 = 0; s2 < S && s2 < kJR; ++s2) facc = facc + __shfl(pw, (lane & ~7) + s2, 64);
        if (S > kJR) facc = facc + slot_term(kJR);
        const int64_t d = (int64_t)(wg + t * G) * kJR + row;
        if (s == 0 && d < Hd) {
            uint32_t yb = bf16_rne(facc);
            if (resid) yb = bf16_rne(bf16_to_f32(resid[d]) + bf16_to_f32(yb));
            Y[d] = (uint16_t)yb;
        }
    }
}

// Staging of the down activation pairs of compute wave (gam, p): pair p of h[q] for its slots.
constexpr int kMaxQ = (kMaxSlots + kGroups - 1) / kGroups;
__device__ __forceinline__ void dn_load_h(uint4 (&xv)[kMaxQ], const uint16_t* Hin, int S, int I, int gam, int p,
                                          int lane) {
    const __amdgpu_buffer_rsrc_t hr = buf_rsrc(Hin, (uint32_t)S * (uint32_t)I * 2u);
#pragma unroll
    for (int i = 0; i < kMaxQ; ++i) {
        const int q = gam + kGroups * i;
        xv[i] = buf_load16(hr, q < S ? (uint32_t)q * (uint32_t)I * 2u + (uint32_t)p * 1024u + 16u * (uint32_t)lane : kOOB);
    }
}
__device__ __forceinline__ void dn_stage_h(const uint4 (&xv)[kMaxQ], uint8_t* s_stage, int S, int gam, int p, int lane) {
#pragma unroll
    for (int i = 0; i < kMaxQ; ++i) {
        const int q = gam + kGroups * i;
        if (q < S) stage_pair(xv[i], s_stage + (uint32_t)(4 * q + p) * kStgBytes, lane);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// x pair pr into registers: staged, then the diagonal operands and sums read back.
__device__ __forceinline__ void x_operands(const uint4& xv, uint8_t* st, int lane, u32x4_t (&A)[8], float2& as) {
    const int n = lane & 15, g = lane >> 4, h = n >> 3;
    stage_pair(xv, st, lane);
#pragma unroll
    for (int i = 0; i < 8; ++i) A[i] = u32x4_t{0u, 0u, 0u, 0u};
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    pair_operands(lds_addr(st), g, n, h, A, as);
}

// ------------------------------------------------------------------ gate/up
template <int R, int NS, int Q, int CW, uint32_t POL>
__global__ __launch_bounds__(64 * (kNCW + CW)) void k_moe_gu_p(Stack Gs, Stack Us, Stack Ds, MoeRoute route, int E,
                                                            int topk, const uint16_t* __restrict__ X,
                                                            uint16_t* __restrict__ Hout, int I, int njobs, int64_t Hd) {
    constexpr int RJ = 2 * R, np = 4 * R, nsb = 8 * R;
    extern __shared__ __align__(16) uint8_t s_dyn[];   // ring | staged pairs
    __shared__ float s_red[kMaxJobs * kRedJob];
    __shared__ uint32_t s_cnt[kMaxJobs * kMaxRJ], s_read[kMaxJobs * kMaxRJ], s_done[kMaxJobs];
    __shared__ __align__(16) uint32_t r_keys[kRouteMaxE];
    __shared__ uint32_t r_win[kRouteMaxTopk];
    __shared__ __align__(16) uint8_t s_pf[1024];   // target of the down-leg prefetch (never read)
    uint8_t* const s_stage = s_dyn + NS * kSlot;
    const Ring rg{s_dyn, s_cnt, s_read, s_done, s_red};
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x, G = gridDim.x;
    const int T = (njobs - wg + G - 1) / G;   // <= kMaxJobs
    const int it8 = I / kJR;
    const int gam = w >> 2, p = w & 3, pr = 4 * gam + p;
    for (int i = tid; i < kMaxJobs * kMaxRJ; i += blockDim.x) s_cnt[i] = s_read[i] = 0u;
    if (tid < kMaxJobs) s_done[tid] = 0u;

    // this wave's activation pair goes out before the routing
    uint4 xv = make_uint4(0u, 0u, 0u, 0u);
    if (w < kNCW && pr < np) xv = buf_load16(buf_rsrc(X, (uint32_t)nsb * 512u), (uint32_t)pr * 1024u + 16u * (uint32_t)lane);
    // routing decision (its barriers also publish the zeroed counters); workgroup 0 forms the
    // slot weights below, once its copies are in flight
    route_workgroup(route.logits, E, topk, route.scale_bits, r_keys, r_win, nullptr, nullptr, false);

    if (w >= kNCW) {   // ---- copy wave c
        const int c = w - kNCW;
        const int ev = slot_experts(r_win, topk, E, lane);
        GuCursor gc;
        gc.start(c, wg, it8, RJ, G);
        copy_ring<NS, Q, CW, kLoads, kReaders>(c, T * RJ, s_cnt, s_read, [&](int u) {
            gu_issue<R, POL>(gc, ev, Gs, Us, topk, s_dyn + (uint32_t)(u % NS) * kSlot, lane);
            gc.advance(CW, it8, RJ, G);
        });
        // the first rounds of the down leg's workgroup wg (output rows 8 wg .., slots 0, 1, ...)
        // into the caches while this workgroup's last sets compute
        const int64_t d0 = (int64_t)wg * kJR;
        if (d0 < Hd) {
            const int nvalid = (int)(Hd - d0 < kJR ? Hd - d0 : kJR);
            const uint32_t off = (uint32_t)(lane & 7) * kRoundRow + 16u * (uint32_t)(lane >> 3);
            for (int q = c; q < kDnPrefetch && q < (Ds.shared ? topk + 1 : topk); q += CW) {
                const __amdgpu_buffer_rsrc_t wr = buf_rsrc(Ds.slot(ev, q, topk) + d0 * (int64_t)kRoundRow,
                                                           (uint32_t)nvalid * kRoundRow);
#pragma unroll
                for (int j = 0; j < kLoads; ++j) lds_dma16<0>(wr, s_pf, off + 128u * j);
            }
            __builtin_amdgcn_s_waitcnt(kWaitVm0);   // no copy into this workgroup's LDS outlives it
        }
        return;
    }
    if (wg == 0 && w == 0) {   // publish the decision for the down leg and the caller
        int32_t sl;
        uint16_t swl;
        route_weights_wave(lane < topk ? r_win[lane] : 0u, topk, route.scale_bits, lane, sl, swl);
        if (lane < topk) {
            route.sel_pub[lane] = sl;
            route.selw_pub[lane] = swl;
            if (route.sel_api) route.sel_api[lane] = sl;
            if (route.selw_api) route.selw_api[lane] = swl;
        }
    }
    if (pr >= np) return;
    // ---- compute wave (gam, p): pair pr of x, operands in registers
    u32x4_t A[8];
    float2 as;
    const int e = pair_exponent(xv);
    x_operands16(xv, s_stage + (uint32_t)pr * kStgBytes, lane, e, A, as);
    const float seed_hi = -1024.0f * __builtin_ldexpf(as.y, -e), hscale = __builtin_ldexpf(1.0f, e - 4);
    int seen = -1;
    gu_jobs<R, NS>(rg, T, 0, wg, G, it8, I, gam, p, A, as, seed_hi, hscale, hdr_sel(lane >> 4), code_k(), code_kh(),
                   seen, Hout, lane);
}

// ------------------------------------------------------------------ down
template <int NS, int Q, int CW, uint32_t POL>
__global__ __launch_bounds__(64 * (kNCW + CW)) void k_moe_down_p(Stack Ds, const int32_t* __restrict__ sel,
                                                              const uint16_t* __restrict__ selw, int E, int topk, int S,
                                                              const uint16_t* __restrict__ Hin, int I, int64_t Hd,
                                                              uint16_t* __restrict__ Y,
                                                              const uint16_t* __restrict__ resid, int njobs) {
    extern __shared__ __align__(16) uint8_t s_dyn[];   // ring | staged pairs [slot][pair]
    __shared__ float s_red[kMaxJobs * kRedJob];         // [job][slot][row][pair]
    __shared__ uint32_t s_cnt[kMaxJobs * kMaxRJ], s_read[kMaxJobs * kMaxRJ], s_done[kMaxJobs];
    uint8_t* const s_stage = s_dyn + NS * kSlot;
    const Ring rg{s_dyn, s_cnt, s_read, s_done, s_red};
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x, G = gridDim.x;
    const int T = (njobs - wg + G - 1) / G;   // <= kMaxJobs
    const int gam = w >> 2, p = w & 3;
    for (int i = tid; i < kMaxJobs * kMaxRJ; i += blockDim.x) s_cnt[i] = s_read[i] = 0u;
    if (tid < kMaxJobs) s_done[tid] = 0u;

    // the activation pairs of this wave's slots go out first
    uint4 xv[kMaxQ];
    if (w < kNCW) dn_load_h(xv, Hin, S, I, gam, p, lane);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // counters initialised

    if (w >= kNCW) {   // ---- copy wave c: lane s holds slot s's expert
        const int c = w - kNCW;
        const int ev = lane < topk ? (sel[lane] < 0 ? 0 : (sel[lane] >= E ? E - 1 : sel[lane])) : 0;
        DnCursor dc;
        dc.start(c, S, wg, G);
        copy_ring<NS, Q, CW, kLoads, kReaders>(c, T * S, s_cnt, s_read, [&](int u) {
            dn_issue<POL>(dc, ev, Ds, topk, Hd, s_dyn + (uint32_t)(u % NS) * kSlot, lane);
            dc.advance(CW, S, G);
        });
        return;
    }
    // ---- compute wave (gam, p): pair p of slots gam, gam + 3, ...
    dn_stage_h(xv, s_stage, S, gam, p, lane);
    int seen = -1;
    dn_jobs<NS>(rg, T, 0, S, topk, wg, G, Hd, gam, p, lds_addr(s_stage), hdr_sel(lane >> 4), code_k(), seen, selw, Y,
                resid, lane);
}

// Ring slots, rounds in flight per copy wave, copy waves (measured: 1 or 2 copy waves, 4 to 7
// rounds each, are within 1 us of each other; these were the fastest).  The ring takes more
// than half the CU's LDS, so the workgroups spread one per CU.
// With a ninth (shared) slot the down leg's staged pairs leave room for 11 slots.
constexpr int kGuNS = 12, kGuQ = 5, kGuCW = 2;
constexpr int kDnNS = 12, kDnNS9 = 11, kDnQ = 7, kDnCW = 1;

size_t gu_lds(int R) { return (size_t)kGuNS * kSlot + (size_t)(4 * R) * kStgBytes; }
size_t dn_lds(int ns, int S) { return (size_t)ns * kSlot + (size_t)(4 * S) * kStgBytes; }

}  // namespace

bool moe_persist_supported(int64_t E, int topk, int nslots, int64_t H, int64_t I) {
    if (topk < 1 || topk > kMaxRouted || (nslots != topk && nslots != topk + 1)) return false;
    if (E < 1 || E > kRouteMaxE || topk > E) return false;
    if (H % 2048 != 0 || H < 2048 || H > 6144 || I != 2048) return false;
    if ((E + 7) / 8 * 8 > 64 * (kNCW + 1)) return false;   // in-kernel routing: one key per thread
    const int64_t cus = device_cu_count();
    const int64_t gu_jobs = (int64_t)nslots * (I / kJR), dn_jobs = (H + kJR - 1) / kJR;
    return gu_jobs <= kMaxJobs * cus && dn_jobs <= kMaxJobs * cus;
}

hipError_t launch_moe_gateup_persist(const uint8_t* G, const uint8_t* U, const uint8_t* shG, const uint8_t* shU,
                                     const uint8_t* D, const uint8_t* shD, const MoeRoute& route, int topk, int nslots,
                                     int64_t E, int64_t H, int64_t I, const uint16_t* x, uint16_t* h, hipStream_t st) {
    if (!moe_persist_supported(E, topk, nslots, H, I) || !route.logits || (nslots > topk && (!shG || !shU)))
        return hipErrorInvalidValue;
    const int R = (int)(H / 2048);
    const int64_t rb = row_bytes(T_Q4_K, H);
    const Stack Gs{G, shG, rb * I}, Us{U, shU, rb * I};
    const Stack Ds{D, nslots > topk ? shD : nullptr, row_bytes(T_Q4_K, I) * H};
    const int njobs = (int)(nslots * (I / kJR));
    const int cus = device_cu_count();
    const int tpw = (njobs + cus - 1) / cus;
    const int G2 = (njobs + tpw - 1) / tpw;
    const dim3 grid(G2), block(64 * (kNCW + kGuCW));
#define AIPU_GU(RV)                                                                                              \
    if (R == RV) {                                                                                               \
        hipLaunchKernelGGL((k_moe_gu_p<RV, kGuNS, kGuQ, kGuCW, kNT>), grid, block, gu_lds(RV), st, Gs, Us, Ds, route, \
                           (int)E, topk, x, h, (int)I, njobs, H);                                                \
        return hipGetLastError();                                                                                \
    }
    AIPU_GU(1) AIPU_GU(2) AIPU_GU(3)
#undef AIPU_GU
    return hipErrorInvalidValue;
}

hipError_t launch_moe_down_persist(const uint8_t* D, const uint8_t* shD, const int32_t* sel, const uint16_t* selw,
                                   int topk, int nslots, int64_t E, int64_t H, int64_t I, const uint16_t* h,
                                   uint16_t* y, const uint16_t* resid, hipStream_t st) {
    if (!moe_persist_supported(E, topk, nslots, H, I) || (nslots > topk && !shD)) return hipErrorInvalidValue;
    const int64_t rb = row_bytes(T_Q4_K, I);
    const Stack Ds{D, shD, rb * H};
    const int njobs = (int)((H + kJR - 1) / kJR);
    const int cus = device_cu_count();
    const int tpw = (njobs + cus - 1) / cus;
    const int G2 = (njobs + tpw - 1) / tpw;
    const dim3 grid(G2), block(64 * (kNCW + kDnCW));
    if (nslots <= kMaxRouted)
        hipLaunchKernelGGL((k_moe_down_p<kDnNS, kDnQ, kDnCW, 0>), grid, block, dn_lds(kDnNS, nslots), st, Ds, sel, selw,
                           (int)E, topk, nslots, h, (int)I, H, y, resid, njobs);
    else
        hipLaunchKernelGGL((k_moe_down_p<kDnNS9, kDnQ, kDnCW, 0>), grid, block, dn_lds(kDnNS9, nslots), st, Ds, sel,
                           selw, (int)E, topk, nslots, h, (int)I, H, y, resid, njobs);
    return hipGetLastError();
}

// Whether a bounded wait in this file's kernels gave up since the last call (then cleared).
hipError_t wait_gave_up_moe_persist(uint32_t* flag) { return take_wait_gave_up(flag); }

}  // namespace aipu
