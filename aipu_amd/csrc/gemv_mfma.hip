// Matrix-core Q4_K GEMV kernels (tolerance mode): the plain GEMV for M = 1..8 activation
// rows, and the MoE expert legs (gate/up with the fused h = bf16(silu(g) * u) epilogue, and
// down with the slot-ordered combine).  The per-tile arithmetic is in mfma_gemv.hpp.
//
// Workgroup.  A workgroup owns T tiles of 16 rows (T = 1 plain, 2 gate/up, nslots down) and
// splits each tile's K into KP equal parts of bpk blocks; wave w computes part w % KP of
// tile w / KP, so W = T * KP waves.  The activations are staged once per workgroup in LDS
// in the MFMA operand order.  The MoE legs (k_gemv1, k_mfma_gemv) reduce per-wave partial
// sums across the wave's four K-groups with two cross-lane adds, then across the KP parts in
// fixed order through LDS; the plain and batched-union kernels for M = 2..8 (k_gemvs, k_gemvm)
// keep every block term and sum them in the fast-mode order of mfma_gemv.hpp, the order of the
// single-row kernel (gemv_persist.hip), so a row of a batch equals its single-row result.
// Every result is deterministic.
//
// Memory order.  Every thread issues its activation loads first, then the wave's first PD
// blocks of weights (buffer loads, streaming cache policy), and only then waits for the
// activations: vector loads return in order, so the staging never waits for the weight
// stream.  The block loop is software pipelined PD deep; loads that fall past the wave's
// blocks or past the tile's valid rows use an out-of-range buffer offset, which reads zero
// without a memory access, so every load is unconditional and the waits are static.
#include <type_traits>

#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"
#include "mfma_gemv.hpp"
#include "route.hpp"

namespace aipu {

using namespace mg;

namespace {

// Problems that declare kCanon = true sum their outputs in the fast-mode order (k_gemv1).
template <class P, class = void>
struct CanonOrder {
    static constexpr bool value = false;
};
template <class P>
struct CanonOrder<P, std::void_t<decltype(P::kCanon)>> {
    static constexpr bool value = P::kCanon;
};

constexpr int kXL = 8;          // activation pieces (16 B) staged per thread, at most
constexpr int kMaxW = 8;        // waves per workgroup
constexpr int64_t kMaxLds = 64 * 1024;

struct TileRef {
    const uint8_t* base;   // row 0 of the tile
    int nvalid;            // rows of the tile that exist (the rest read as zero)
    int act;               // which staged activation the tile multiplies
};

// ------------------------------------------------------------------ problems
// Plain GEMV: tile = 16 consecutive rows of W, activation rows x[M][K].
template <int MR>
struct ProbPlain {
    // k_gemv1 forms the output in the fast-mode order of mfma_gemv.hpp (block terms, pair sums,
    // the balanced tree), the order of every other single-row and batch kernel
    static constexpr bool kCanon = true;
    const uint8_t* W;
    int64_t N, rb;
    uint16_t* Y;
    float* Yf;
    int64_t ystride;   // N of the full output (tiles of a mixed call write a column slice)
    int M;
    static constexpr bool kRoutes = false;
    static constexpr bool kShareAct = false;
    static constexpr int kTiles = 1;
    static constexpr uint32_t kPolicy = kNT;   // weights stream past the caches
    static constexpr int kRows = MR;
    __device__ void setup(int, uint32_t*, uint32_t*, int32_t*, uint16_t*) {}
    __device__ bool active(int) const { return true; }
    __device__ const uint16_t* act(int, const uint16_t* X) const { return X; }
    __device__ TileRef tile(int wg, int) const {
        const int64_t r0 = (int64_t)wg * kTR;
        const int64_t nv = N - r0;
        return TileRef{W + r0 * rb, (int)(nv < kTR ? nv : kTR), 0};
    }
    __device__ void finish(int wg, const float* red, int KP, int tid) const {
        if (tid >= kTR * MR) return;
        const int n = tid / MR, r = tid % MR;
        const int64_t row = (int64_t)wg * kTR + n;
        if (r >= M || row >= N) return;
        float v = 0.f;
        for (int k = 0; k < KP; ++k) v += red[(k * kTR + n) * MR + r];
        Y[r * ystride + row] = (uint16_t)bf16_rne(v);
        if (Yf) Yf[r * ystride + row] = v;
    }
    // one output (row n of the tile, activation row r) of the small-batch kernel
    __device__ void store(int wg, int n, int r, float v) const {
        const int64_t row = (int64_t)wg * kTR + n;
        if (r >= M || row >= N) return;
        Y[r * ystride + row] = (uint16_t)bf16_rne(v);
        if (Yf) Yf[r * ystride + row] = v;
    }
};

__device__ __forceinline__ int routed_expert(const int32_t* sel, int s, int E) {
    const int e = sel[s];
    return e < 0 ? 0 : (e >= E ? E - 1 : e);
}

// MoE gate/up: workgroup (slot, 16-row tile of I); tile 0 = gate rows, tile 1 = up rows of
// the slot's expert (slot topk = the shared expert).  h[slot][i] = bf16(silu(g) * u).
// With route.logits set, every workgroup first computes the routing decision itself from
// the router logits (route.hpp) -- no workgroup waits for another -- and workgroup 0
// publishes it for the down leg and the caller.
struct ProbGateUp {
    const uint8_t *G, *U, *shG, *shU;
    MoeRoute route;
    int topk, E, itiles;
    int64_t rb, ebytes;
    uint16_t* h;
    int64_t I;
    int eid;   // expert of this workgroup's slot (setup)
    static constexpr bool kRoutes = true;
    // the gate and up tiles of a workgroup read the same activations: the two waves of each
    // K part share one staging slot (written by the gate wave)
    static constexpr bool kShareAct = true;
    static constexpr uint32_t kPolicy = 0;   // default caching: measured faster for the MoE legs
    __device__ void setup(int wg, uint32_t* keys, uint32_t* win, int32_t* sel, uint16_t* selw) {
        const int s = wg / itiles;
        if (route.logits) {
            // workgroup 0 also forms the slot weights and publishes the decision
            route_workgroup(route.logits, E, topk, route.scale_bits, keys, win, sel, selw, wg == 0);
            if (wg == 0 && (int)threadIdx.x < topk) {
                route.sel_pub[threadIdx.x] = sel[threadIdx.x];
                route.selw_pub[threadIdx.x] = selw[threadIdx.x];
                if (route.sel_api) route.sel_api[threadIdx.x] = sel[threadIdx.x];
                if (route.selw_api) route.selw_api[threadIdx.x] = selw[threadIdx.x];
            }
            const int e = s < topk ? (int)(0xFFFFu - (win[s] & 0xFFFFu)) : 0;
            eid = __builtin_amdgcn_readfirstlane(e < 0 ? 0 : (e >= E ? E - 1 : e));
        } else {
            eid = s < topk ? __builtin_amdgcn_readfirstlane(routed_expert(route.sel, s, E)) : 0;
        }
    }
    __device__ TileRef tile(int wg, int t) const {
        const int s = wg / itiles, it = wg - s * itiles;
        const uint8_t* base;
        if (s < topk) base = (t ? U : G) + (int64_t)eid * ebytes;
        else base = t ? shU : shG;
        return TileRef{base + (int64_t)it * kTR * rb, kTR, 0};
    }
    __device__ void finish(int wg, const float* red, int KP, int tid) const {
        if (tid >= kTR) return;
        const int s = wg / itiles, it = wg - s * itiles;
        float g = 0.f, u = 0.f;
        for (int k = 0; k < KP; ++k) {
            g += red[k * kTR + tid];
            u += red[(KP + k) * kTR + tid];
        }
        const uint32_t gb = bf16_rne(g), ub = bf16_rne(u);
        h[(int64_t)s * I + (int64_t)it * kTR + tid] =
            (uint16_t)bf16_rne(bf16_to_f32(glm_silu_bf16(gb)) * bf16_to_f32(ub));
    }
};

// MoE down: workgroup = 16-row tile of H; tile s = slot s (its expert's rows, against
// h[s]).  The slots are combined in slot order
//     facc = f32(facc + f32(w_s * bf16(y_s)))   (tools/glm_model_q4k_ref.py:799-809)
// with w = 1 for the shared slot; passthrough (one expert, no routing) writes bf16(y_0).
struct ProbDown {
    const uint8_t *D, *shD;
    const int32_t* sel;
    const uint16_t* selw;
    int topk, nslots, E, passthrough;
    int64_t H, rb, ebytes;
    uint16_t* Y;
    // Split combine (more slots than one workgroup's waves): the first launch leaves the
    // fp32 running sum in acc_out, the second starts from acc_in.  resid (nullable) is added
    // after the bf16 rounding: Y = bf16(resid + bf16(facc)) (the decoder block's residual).
    const float* acc_in = nullptr;
    float* acc_out = nullptr;
    const uint16_t* resid = nullptr;
    static constexpr bool kRoutes = false;
    static constexpr bool kShareAct = false;
    static constexpr uint32_t kPolicy = 0;   // default caching: measured faster for the MoE legs
    __device__ void setup(int, uint32_t*, uint32_t*, int32_t*, uint16_t*) {}
    __device__ TileRef tile(int wg, int t) const {
        const int64_t d0 = (int64_t)wg * kTR;
        const uint8_t* base = t < topk ? D + (int64_t)routed_expert(sel, t, E) * ebytes : shD;
        const int64_t nv = H - d0;
        return TileRef{base + d0 * rb, (int)(nv < kTR ? nv : kTR), t};
    }
    __device__ void finish(int wg, const float* red, int KP, int tid) const {
        if (tid >= kTR) return;
        const int64_t d = (int64_t)wg * kTR + tid;
        if (d >= H) return;
        float facc = acc_in ? acc_in[d] : 0.f;
        for (int s = 0; s < nslots; ++s) {
            float ys = 0.f;
            for (int k = 0; k < KP; ++k) ys += red[(s * KP + k) * kTR + tid];
            if (passthrough) {
                Y[d] = (uint16_t)bf16_rne(ys);
                return;
            }
            const float yb = bf16_to_f32(bf16_rne(ys));
            const float p = s < topk ? bf16_to_f32(selw[s]) * yb : yb;
            facc = facc + p;
        }
        if (acc_out) {
            acc_out[d] = facc;
            return;
        }
        uint32_t yb = bf16_rne(facc);
        if (resid) yb = bf16_rne(bf16_to_f32(resid[d]) + bf16_to_f32(yb));
        Y[d] = (uint16_t)yb;
    }
};

// ------------------------------------------------------------------ kernel
struct Plan {
    int KP, bpk, PD, W, nact;
    int64_t lds;
};

template <int MR>
__device__ __forceinline__ void lds_sums(const uint8_t* smem, uint32_t off, float (&lo)[MR], float (&hi)[MR]) {
    if constexpr (MR == 1) {
        const float2 v = *(const float2*)(smem + off);
        lo[0] = v.x;
        hi[0] = v.y;
    } else if constexpr (MR == 2) {
        const float4 v = *(const float4*)(smem + off);
        lo[0] = v.x;
        lo[1] = v.y;
        hi[0] = v.z;
        hi[1] = v.w;
    } else {
        const float4 a = *(const float4*)(smem + off);
        const float4 b = *(const float4*)(smem + off + 16);
        lo[0] = a.x;
        lo[1] = a.y;
        lo[2] = a.z;
        lo[3] = a.w;
        hi[0] = b.x;
        hi[1] = b.y;
        hi[2] = b.z;
        hi[3] = b.w;
    }
}

__device__ __forceinline__ u32x4_t lds128(const uint8_t* smem, uint32_t off) {
    const uint4 v = *(const uint4*)(smem + off);
    return u32x4_t{v.x, v.y, v.z, v.w};
}

template <int MR, int PD, class Prob>
__global__ __launch_bounds__(kMaxW * 64) void k_mfma_gemv(Prob pb0, const uint16_t* __restrict__ X, int64_t xstride,
                                                          uint32_t xbytes, int K, int M, int nact, int KP, int bpk) {
    static_assert(MR == 1 || MR == 2 || MR == 4, "MR must be 1, 2 or 4");
    using L = ActLayout<MR>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nthr = blockDim.x;
    const int nsb = K / QK_K;
    const int wg = blockIdx.x;
    const uint32_t abytes = (uint32_t)nsb * L::kEntriesPerBlock * 16;   // A entries of one activation
    const uint32_t aoff0 = L::kZeroBytes;
    const uint32_t soff0 = aoff0 + (uint32_t)nact * abytes;
    const uint32_t sbytes = (uint32_t)nsb * L::kSumsPerBlock * 4;
    float* red = (float*)(smem + soff0 + (uint32_t)nact * sbytes);

    // ---- 1. activation loads: piece q = (act*MR + m) * ppr + p, 8 bf16 at position 8p
    const int ppr = nsb * 32;
    const int total = nact * MR * ppr;
    const float inv_ppr = 1.0f / (float)ppr;
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, xbytes);
    uint4 xv[kXL];
#pragma unroll
    for (int i = 0; i < kXL; ++i) {
        const int q = tid + i * nthr;
        const int rowid = (int)(((float)q + 0.5f) * inv_ppr);
        const int p = q - rowid * ppr;
        const int a = rowid / MR, m = rowid - a * MR;
        const bool valid = q < total && m < M;
        const uint32_t off = valid ? 2u * (uint32_t)((int64_t)a * xstride + (int64_t)m * K + 8 * p) : kOOB;
        xv[i] = buf_load16(xr, off);
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. the wave's tile and its first PD blocks of weights
    Prob pb = pb0;
    if constexpr (Prob::kRoutes) {
        __shared__ __align__(16) uint32_t r_keys[kRouteMaxE];
        __shared__ uint32_t r_win[kRouteMaxTopk];
        __shared__ int32_t r_sel[kRouteMaxTopk];
        __shared__ uint16_t r_selw[kRouteMaxTopk];
        pb.setup(wg, r_keys, r_win, r_sel, r_selw);
    }
    const int tt = w / KP, kp = w - tt * KP;
    const TileRef tr = pb.tile(wg, tt);
    const int64_t rb = (int64_t)nsb * 144;
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(tr.base, (uint32_t)(tr.nvalid * rb));
    const int n = lane & 15, g = lane >> 4;
    const uint32_t row_off = (uint32_t)(n * rb);   // rows >= nvalid land out of range -> zeros
    const int kb0 = kp * bpk;
    Raw buf[PD];
#pragma unroll
    for (int j = 0; j < PD; ++j) buf[j] = raw_load(wr, row_off + (uint32_t)(kb0 + j) * 144u, g);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. stage: zero region, permuted activations, sub-block sums
    for (int i = tid; i < L::kZeroBytes / 16; i += nthr) ((uint4*)smem)[i] = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < kXL; ++i) {
        const int q = tid + i * nthr;
        const int rowid = (int)(((float)q + 0.5f) * inv_ppr);
        const int p = q - rowid * ppr;
        const int a = rowid / MR, m = rowid - a * MR;
        // sum of the piece's 8 activations, then of the 4 pieces of its sub-block (a quad)
        const uint32_t ones = 0x3F803F80u;
        float s = 0.f;
        s = dot2(xv[i].x, ones, s);
        s = dot2(xv[i].y, ones, s);
        s = dot2(xv[i].z, ones, s);
        s = dot2(xv[i].w, ones, s);
        s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0xB1, 0xF, 0xF, false));
        s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x4E, 0xF, 0xF, false));
        if (q < total) {
            const int b = p >> 5, gg = (p >> 3) & 3, t = p & 7;
            const uint32_t e = (uint32_t)((b * 8 + t) * 4 + gg) * MR + m;
            *(u32x4_t*)(smem + aoff0 + (uint32_t)a * abytes + 16u * e) = act_perm(xv[i]);
            if ((p & 3) == 0) {
                const int h = (p >> 2) & 1;
                ((float*)(smem + soff0 + (uint32_t)a * sbytes))[((b * 4 + gg) * 2 + h) * MR + m] = s;
            }
        }
    }
    __syncthreads();

    // ---- 4. block loop
    const int mm = n - 4 * g;
    const bool diag = mm >= 0 && mm < MR;
    const uint32_t alane = diag ? aoff0 + (uint32_t)tr.act * abytes + 16u * (uint32_t)(g * MR + mm) : 0u;
    const uint32_t ablk = diag ? (uint32_t)L::kEntriesPerBlock * 16u : 0u;
    const uint32_t slane = soff0 + (uint32_t)tr.act * sbytes + 4u * (uint32_t)(g * 2 * MR);
    const HdrSel hs = hdr_sel(g);
    const CodeK ck = code_k();
    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.f;
    // Accumulator rows r >= MR multiply all-zero activation rows and stay 0; only rows < MR
    // are re-seeded per block.
    f32x4_t dlo = {0.f, 0.f, 0.f, 0.f}, dhi = {0.f, 0.f, 0.f, 0.f};

    for (int s0 = 0; s0 < bpk; s0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; ++j) {
            const int b = kb0 + s0 + j;
            const Raw& R = buf[j];
            const uint32_t ab = alane + ablk * (uint32_t)b;
            u32x4_t A[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) A[t] = lds128(smem, ab + 16u * (uint32_t)(t * 4 * MR));
            float alo[MR], ahi[MR];
            lds_sums<MR>(smem, slane + 4u * (uint32_t)(b * 8 * MR), alo, ahi);
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                dlo[r] = -kCodeBiasF * alo[r];
                dhi[r] = -kCodeBiasF * ahi[r];
            }
            const uint32_t qd[8] = {R.q0.x, R.q0.y, R.q0.z, R.q0.w, R.q1.x, R.q1.y, R.q1.z, R.q1.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                dlo = mfma(A[t], codes_lo(qd[2 * t], qd[2 * t + 1], ck), dlo);
                dhi = mfma(A[4 + t], codes_hi(qd[2 * t], qd[2 * t + 1], ck), dhi);
            }
            const Hdr H = hdr_decode(R.h, hs);
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                const float t1 = __builtin_fmaf(H.sc1, dhi[r], H.sc0 * dlo[r]);
                const float v = __builtin_fmaf(H.m1, ahi[r], H.m0 * alo[r]);
                acc[r] = __builtin_fmaf(H.d, t1, acc[r]);
                acc[r] = __builtin_fmaf(-H.dm, v, acc[r]);
            }
            // refill this slot right away (the loads must not sink to the end of the group)
            const int sn = s0 + j + PD;
            buf[j] = raw_load(wr, sn < bpk ? row_off + (uint32_t)(kb0 + sn) * 144u : kOOB, g);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- 5. reduce over the four K-groups (lanes n, n+16, n+32, n+48), then across parts
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        acc[r] += __shfl_xor(acc[r], 16, 64);
        acc[r] += __shfl_xor(acc[r], 32, 64);
    }
    if (lane < kTR) {
#pragma unroll
        for (int r = 0; r < MR; ++r) red[(w * kTR + lane) * MR + r] = acc[r];
    }
    __syncthreads();
    pb.finish(wg, red, KP, tid);
}

// ------------------------------------------------------- single-row kernel (M = 1)
// Each wave is self-contained: it stages the activations of its own BPK = GS * NG blocks
// and streams its 16 rows of weights group by group (GS blocks per group) into its own LDS
// slice with direct-to-LDS buffer loads, 16 contiguous bytes per lane, so every load
// instruction covers ~1 KB of consecutive row bytes and no byte is fetched twice.  A group
// is copied from LDS into registers before the next group's loads are issued into the same
// slice, so the next group's memory latency overlaps this group's arithmetic.  No barrier
// precedes the block loop; the one barrier is the final reduction across the K parts.
template <int GS>
struct Dma {
    static constexpr int kPieces = 16 * 9 * GS;            // 16-B pieces of 16 rows x GS blocks
    static constexpr int kInsts = (kPieces + 63) / 64;     // 64 lanes x 16 B per instruction
    static constexpr int kBytes = kInsts * 1024;           // LDS slice (the tail lanes write zeros)
};

template <int GS, uint32_t POL = kNT>
__device__ __forceinline__ void dma_group(__amdgpu_buffer_rsrc_t wr, uint8_t* slice, int64_t rb, int blk0, int lane) {
#pragma unroll
    for (int i = 0; i < Dma<GS>::kInsts; ++i) {
        const int j = 64 * i + lane;
        const int row = j / (9 * GS), within = j - row * (9 * GS);
        const uint32_t off = j < Dma<GS>::kPieces ? (uint32_t)(row * rb + (int64_t)blk0 * 144 + 16 * within) : kOOB;
        lds_dma16<POL>(wr, slice + 1024 * i, off);
    }
}

template <int GS, int XI, class Prob, bool kLoop = false>
__global__ __launch_bounds__(kMaxW * 64) void k_gemv1(Prob pb0, const uint16_t* __restrict__ X, int64_t xstride,
                                                      uint32_t xbytes, int K, int KP, int NG, int tpw) {
    // Separate LDS objects for the direct-to-LDS weight slices (dynamic) and for everything
    // the waves write themselves (static), so the compiler can see that the staging writes
    // do not alias weight loads still in flight and does not make them wait for those.
    constexpr int kBpkMax = 2 * XI;             // activation pieces per wave <= 64 * XI
    constexpr uint32_t kActWave = kBpkMax * 544;
    constexpr int kSlots = Prob::kShareAct ? kMaxW / 2 : kMaxW;   // activation staging slots
    __shared__ __align__(16) uint8_t s_act[kSlots * kActWave];
    __shared__ float red[(kLoop ? 2 : 1) * kMaxW * kTR];   // double-buffered across a workgroup's tiles
    // fast-mode order: every block term of the tile, [row][block] (one tile per workgroup)
    constexpr bool kCanon = CanonOrder<Prob>::value;
    __shared__ float bterm[kCanon ? kTR * kMaxW * kBpkMax : 1];
    extern __shared__ __align__(16) uint8_t s_w[];
    const int BPK = GS * NG;
    const int XP = BPK * 32;
    const uint32_t kA = (uint32_t)BPK * 512;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: the copies take a scalar LDS base
    const int nsb = K / QK_K;
    const int wg = blockIdx.x;
    uint8_t* wW = s_w + (uint32_t)w * Dma<GS>::kBytes;

    // A workgroup computes tiles t0 .. t0 + tpw - 1 (tiles that share the routing decision and
    // the activations); the first weight group of tile t + 1 is copied while tile t finishes.
    if constexpr (!kLoop) tpw = 1;   // one tile per workgroup: the loop folds away
    const int t0 = wg * tpw;
    Prob pb = pb0;
    if constexpr (Prob::kRoutes) {   // routing decision (before any weight address is known)
        __shared__ __align__(16) uint32_t r_keys[kRouteMaxE];
        __shared__ uint32_t r_win[kRouteMaxTopk];
        __shared__ int32_t r_sel[kRouteMaxTopk];
        __shared__ uint16_t r_selw[kRouteMaxTopk];
        pb.setup(t0, r_keys, r_win, r_sel, r_selw);
    }
    const int tt = w / KP, kp = w - tt * KP;
    const TileRef tr = pb.tile(t0, tt);
    const int kb0 = kp * BPK;
    const int64_t rb = (int64_t)nsb * 144;
    uint8_t* wA = s_act + (uint32_t)(Prob::kShareAct ? kp : w) * kActWave;
    float* wS = (float*)(wA + kA);
    const bool stager = !Prob::kShareAct || tt == 0;

    // 1. this wave's activations, then 2. its first group of weights
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, xbytes);
    const uint32_t xbase = 2u * (uint32_t)((int64_t)tr.act * xstride + (int64_t)kb0 * QK_K);
    uint4 xv[XI];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int q = lane + 64 * i;
        xv[i] = buf_load16(xr, q < XP && stager ? xbase + 16u * q : kOOB);
    }
    __amdgpu_buffer_rsrc_t wr = buf_rsrc(tr.base, (uint32_t)(tr.nvalid * rb));
    dma_group<GS, Prob::kPolicy>(wr, wW, rb, kb0, lane);
    __builtin_amdgcn_sched_barrier(0);

    // 3. stage: A entries, sums (with shared slots, the gate waves stage for both tiles and
    // an LDS-only barrier -- the weight copies stay in flight -- publishes them)
    if (stager) {
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int q = lane + 64 * i;
        const uint32_t ones = 0x3F803F80u;
        float sm = 0.f;
        sm = dot2(xv[i].x, ones, sm);
        sm = dot2(xv[i].y, ones, sm);
        sm = dot2(xv[i].z, ones, sm);
        sm = dot2(xv[i].w, ones, sm);
        sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
        sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x4E, 0xF, 0xF, false));
        if (q < XP) {
            const int bb = q >> 5, gg = (q >> 3) & 3, t = q & 7;
            *(u32x4_t*)(wA + 16u * (uint32_t)((bb * 8 + t) * 4 + gg)) = act_perm(xv[i]);
            if ((q & 3) == 0) wS[(bb * 4 + gg) * 2 + ((q >> 2) & 1)] = sm;
        }
    }
    }
    if constexpr (Prob::kShareAct) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // 4. block loop
    const int n = lane & 15, g = lane >> 4;
    u32x4_t A[8];   // block-diagonal activation operands: off-diagonal lanes stay zero
#pragma unroll
    for (int t = 0; t < 8; ++t) A[t] = u32x4_t{0u, 0u, 0u, 0u};
    const HdrSel hs = hdr_sel(g);
    const CodeK ck = code_k();
    const uint32_t rrow = (uint32_t)n * (144u * GS);
    f32x4_t dlo = {0.f, 0.f, 0.f, 0.f}, dhi = {0.f, 0.f, 0.f, 0.f};
    for (int ti = 0; ti < tpw; ++ti) {
        const int t = t0 + ti;
        float acc = 0.f;
        for (int gi = 0; gi < NG; ++gi) {
            __builtin_amdgcn_s_waitcnt(kWaitVm0);    // this group's weights are in LDS
            Raw R[GS];
#pragma unroll
            for (int bb = 0; bb < GS; ++bb) {
                const uint8_t* p = wW + rrow + 144u * bb;
                R[bb].h = *(const uint4*)p;
                R[bb].q0 = *(const uint4*)(p + 16 + 32 * g);
                R[bb].q1 = *(const uint4*)(p + 32 + 32 * g);
            }
            if (gi + 1 < NG) {
                regs_consumed(R);   // the slice has been read: refill it
                dma_group<GS, Prob::kPolicy>(wr, wW, rb, kb0 + (gi + 1) * GS, lane);
            } else if (ti + 1 < tpw) {
                regs_consumed(R);   // the next tile's first group
                const TileRef tn = pb.tile(t + 1, tt);
                wr = buf_rsrc(tn.base, (uint32_t)(tn.nvalid * rb));
                dma_group<GS, Prob::kPolicy>(wr, wW, rb, kb0, lane);
            }
#pragma unroll
            for (int bb = 0; bb < GS; ++bb) {
                const int b = gi * GS + bb;   // block index within this wave's part
                a_reads(A, lds_addr(wA + 512u * (uint32_t)b + 16u * (uint32_t)g), diag_mask(1));
                const float2 as = sums_read(wS + (b * 4 + g) * 2);   // no wait on the refill in flight
                if constexpr (kCanon) {
                    // block term: the four K-groups' terms (q4k_block1 from zero is block_term)
                    const float bt = block_sum(q4k_block1(R[bb], A, as, hs, ck, dlo, dhi, 0.0f));
                    if (lane < kTR) bterm[lane * nsb + kb0 + b] = bt;
                } else {
                    acc = q4k_block1(R[bb], A, as, hs, ck, dlo, dhi, acc);
                }
            }
        }
        if constexpr (kCanon) {
            // pair sums and the balanced tree over every block term of the row, on eight lanes
            // per row (canon_sum8)
            __syncthreads();
            for (int i = tid; i < kTR * 8; i += (int)blockDim.x) {
                const int rn = i >> 3, k = i & 7;
                const float y = canon_sum8(nsb, k, [&](int b) { return bterm[rn * nsb + b]; });
                if (k == 0) pb.store(t, rn, 0, y);
            }
            if constexpr (kLoop) __syncthreads();   // read before a next tile writes its terms
            continue;
        }

        // 5. reduce over the four K-groups, then across the K parts (an LDS-only barrier: the
        // next tile's copies stay in flight)
        acc += __shfl_xor(acc, 16, 64);
        acc += __shfl_xor(acc, 32, 64);
        float* rd = red + (ti & 1) * (kMaxW * kTR);
        if (lane < kTR) rd[w * kTR + lane] = acc;
        if constexpr (kLoop) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else __syncthreads();
        pb.finish(t, rd, KP, tid);
    }
}

// ------------------------------------------------- register-weight kernel (M = 5 .. 8)
// Five to eight activation rows (eight rows' staged activations leave no LDS for copying the
// weights), the batched-MoE union legs, and shapes the small-batch plan does not cover.
// One 16-row weight tile per workgroup, its K split over KP waves of BPK blocks each.  A
// wave loads its weight blocks straight into registers (all of them at once), and stages
// only its own K-slice of the MR activation rows in its own LDS region, so no barrier
// precedes the block loop.  Activation rows 4h .. 4h+3 form the block-diagonal operand of
// MFMA set h (lane 16g + n reads row 4h + n - 4g of K-group g), so one set of codes serves
// four rows and lane 16g + n ends with the sums of rows 4h + r in its D registers r.
// LDS layout per wave: operand entries [b][g][m][t] (16 B each; a (b, g, m) group of 8 is
// padded to 144 B so that the 16 diagonal lanes hit distinct banks), the sub-block sums
// [b][g][lo/hi][m] (fp32), and one zero group that the off-diagonal lanes read (plain LDS
// loads on every lane, so the compiler tracks every wait).

template <int MR, int BPK, class Prob>
__global__ __launch_bounds__(kMaxW * 64) void k_gemvm(Prob pb, const uint16_t* __restrict__ X0, int K) {
    constexpr int MRQ = MR < 4 ? MR : 4;   // rows per MFMA set
    constexpr int NH = MR / MRQ;           // MFMA sets (1, or 2 for MR = 8)
    constexpr int kGrp = 144;                       // bytes per (b, g, m) group of 8 entries
    constexpr int kEnt = BPK * 4 * MR * kGrp;       // operand bytes per wave
    constexpr int kSums = BPK * 8 * MR * 4;
    constexpr int kZero = kGrp;                     // zeros read by off-diagonal lanes
    constexpr int kWave = kEnt + kSums + kZero;
    constexpr int kPieces = MR * BPK * 32;   // 16-B activation pieces per wave
    constexpr int kXL = (kPieces + 63) / 64;
    __shared__ __align__(16) uint8_t s_act[kMaxW * kWave];
    static_assert(kTR * MR * kMaxW * BPK * 4 <= kMaxW * kWave, "the block terms fit over the operand entries");
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nsb = K / QK_K;
    const int wg = blockIdx.x;
    if (!pb.active(wg)) return;            // workgroup-uniform: past a data-dependent grid end
    const uint16_t* __restrict__ X = pb.act(wg, X0);
    uint8_t* wA = s_act + (uint32_t)w * kWave;
    float* wS = (float*)(wA + kEnt);
    const int kb0 = w * BPK;
    const int64_t rb = (int64_t)nsb * 144;
    const int n = lane & 15, g = lane >> 4;

    // 1. activations of this wave's K-slice (rows >= M read as zero), 2. its weight blocks
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, (uint32_t)((int64_t)pb.M * K * 2));
    uint4 xv[kXL];
#pragma unroll
    for (int i = 0; i < kXL; ++i) {
        const int q = lane + 64 * i;
        const int m = q / (BPK * 32), p = q - m * (BPK * 32);
        const uint32_t off = q < kPieces ? 2u * (uint32_t)((int64_t)m * K + (int64_t)kb0 * QK_K) + 16u * (uint32_t)p : kOOB;
        xv[i] = buf_load16(xr, off);
    }
    const TileRef tr = pb.tile(wg, 0);
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(tr.base, (uint32_t)(tr.nvalid * rb));
    Raw R[BPK];
#pragma unroll
    for (int b = 0; b < BPK; ++b) R[b] = raw_load(wr, (uint32_t)(n * rb) + (uint32_t)(kb0 + b) * 144u, g);
    __builtin_amdgcn_sched_barrier(0);

    // 3. stage operand entries and sub-block sums, and clear the zero region
    if (lane < kZero / 16) *(u32x4_t*)(wA + kEnt + kSums + 16u * (uint32_t)lane) = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < kXL; ++i) {
        const int q = lane + 64 * i;
        const int m = q / (BPK * 32), p = q - m * (BPK * 32);
        const uint32_t ones = 0x3F803F80u;
        float sm = 0.f;
        sm = dot2(xv[i].x, ones, sm);
        sm = dot2(xv[i].y, ones, sm);
        sm = dot2(xv[i].z, ones, sm);
        sm = dot2(xv[i].w, ones, sm);
        sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
        sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x4E, 0xF, 0xF, false));
        if (q < kPieces) {
            const int bb = p >> 5, gg = (p >> 3) & 3, t = p & 7;
            *(u32x4_t*)(wA + (uint32_t)(kGrp * ((bb * 4 + gg) * MR + m) + 16 * t)) = act_perm(xv[i]);
            if ((p & 3) == 0) wS[((bb * 4 + gg) * 2 + ((p >> 2) & 1)) * MR + m] = sm;
        }
    }

    // 4. block loop
    const int mm = n - 4 * g;
    const bool diag = mm >= 0 && mm < MRQ;
    const HdrSel hs = hdr_sel(g);
    const CodeK ck = code_k();
    u32x4_t A[NH][8];
    float bt[BPK][NH];   // block terms: lane 16i + n holds row n, activation row 4h + i
    f32x4_t dlo[NH], dhi[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) dlo[h] = dhi[h] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint32_t zero_off = (uint32_t)(kEnt + kSums);
#pragma unroll
    for (int b = 0; b < BPK; ++b) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const uint32_t base = diag ? (uint32_t)(kGrp * ((b * 4 + g) * MR + 4 * h + mm)) : zero_off;
#pragma unroll
            for (int t = 0; t < 8; ++t) A[h][t] = lds128(wA, base + 16u * (uint32_t)t);
        }
        float alo[MR], ahi[MR];
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            alo[r] = wS[((b * 4 + g) * 2 + 0) * MR + r];
            ahi[r] = wS[((b * 4 + g) * 2 + 1) * MR + r];
        }
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int r = 0; r < MRQ; ++r) {
                dlo[h][r] = -kCodeBiasF * alo[4 * h + r];
                dhi[h][r] = -kCodeBiasF * ahi[4 * h + r];
            }
        const uint32_t qd[8] = {R[b].q0.x, R[b].q0.y, R[b].q0.z, R[b].q0.w, R[b].q1.x, R[b].q1.y, R[b].q1.z, R[b].q1.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const u32x4_t cl = codes_lo(qd[2 * t], qd[2 * t + 1], ck);
            const u32x4_t cu = codes_hi(qd[2 * t], qd[2 * t + 1], ck);
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                dlo[h] = mfma(A[h][t], cl, dlo[h]);
                dhi[h] = mfma(A[h][4 + t], cu, dhi[h]);
            }
        }
        const Hdr H = hdr_decode(R[b].h, hs);
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            float t[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) t[r] = r < MRQ ? block_term(H, dlo[h][r], dhi[h][r], alo[4 * h + r], ahi[4 * h + r]) : 0.f;
            bt[b][h] = MRQ == 4 ? block_sum4(t[0], t[1], t[2], t[3]) : block_sum2(t[0], t[1]);
        }
    }

    // 5. the block terms of all K parts into LDS (over the operand entries, once every wave
    // is past its block loop), then each output in the fast-mode order
    float* terms = (float*)s_act;   // [n][m][b], b < nsb
    __syncthreads();
    {
        const int i = lane >> 4;   // activation row within the set (MRQ = 2: rows 0, 1 twice)
        if (i < MRQ) {
#pragma unroll
            for (int b = 0; b < BPK; ++b)
#pragma unroll
                for (int h = 0; h < NH; ++h) terms[(n * MR + 4 * h + i) * nsb + kb0 + b] = bt[b][h];
        }
    }
    __syncthreads();
    // eight lanes per output (uniform trip count: every lane takes part in the cross-lane adds)
    const int per = (int)(blockDim.x >> 3);
    for (int o0 = 0; o0 < kTR * MR; o0 += per) {
        const int o = o0 + (tid >> 3), rn = o / MR, m = o - rn * MR;
        const bool valid = o < kTR * MR && m < pb.M;
        const float* te = terms + (valid ? (rn * MR + m) * nsb : 0);
        const float y = canon_sum8(nsb, lane & 7, [&](int b) { return te[b]; });
        if (valid && (lane & 7) == 0) pb.store(wg, rn, m, y);
    }
}

// ------------------------------------------------- small-batch kernel (M = 2 .. 4)
// The single-row kernel's memory plan for up to four activation rows.  A workgroup owns one
// 16-row tile, its K split over KP <= NW waves of GS blocks; each wave copies all its weight
// blocks straight into its LDS slice at once (1 KB of consecutive row bytes per
// instruction) and moves them into registers.  Row m is row 4g + m of the block-diagonal
// operand, so one set of codes (the VALU work of a block) serves all rows and lane 16g + n
// ends with the row-n sums of every row in its D registers.  The operand entries
// ([b][t][g][m & 1], 16 B) sit in two places: rows 0, 1 in the wave's static region, staged
// while the weights are in flight, and rows 2, 3 in the wave's own weight slice, free once
// the blocks are in registers.  The sub-block activation sums stay in registers (each lane
// fetches its own from the staging lanes) and the block terms go through the
// slices.  At K = 6144 eight waves of three blocks take 57,344 + 24,576 B, exactly half the
// CU's LDS, so two workgroups share a CU as in the M = 1 kernel.
constexpr int kSmallMaxRows = 4;

template <int GS, int NW, int MR, class Prob>   // MR = 2: rows 0, 1 only; MR = 4: up to four rows
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(4))) void k_gemvs(
    Prob pb, const uint16_t* __restrict__ X0, int K) {
    constexpr int XP = GS * 32;              // 16-B pieces per activation row and wave
    constexpr int XI = (2 * XP + 63) / 64;   // pieces per lane for a pair of rows
    constexpr uint32_t kPair = GS * 1024u;   // operand entries of a pair of rows
    constexpr uint32_t kRed = kPair;         // block terms [n][column][block], after the entries in the slice
    constexpr int NT = Prob::kTiles;         // tiles per workgroup (the next one copied while one computes)
    constexpr int kCols = 2 * NT > kSmallMaxRows ? 2 * NT : kSmallMaxRows;   // block-term columns per row
    static_assert(kRed + kTR * kCols * GS * 4 <= (uint32_t)Dma<GS>::kBytes, "slice holds a pair and the block terms");
    static_assert(NT == 1 || MR == 2, "a later tile's copy reuses the slice rows 2, 3 would use");
    __shared__ __align__(16) uint8_t s_act[NW * kPair];
    extern __shared__ __align__(16) uint8_t s_w[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: the copies take a scalar LDS base
    const int nsb = K / QK_K;
    const int wg = blockIdx.x;
    if (!pb.active(wg)) return;   // workgroup-uniform: past a data-dependent grid end
    const uint16_t* __restrict__ X = pb.act(wg, X0);
    const int rows = pb.M;   // 1 .. MR
    uint8_t* wA = s_act + (uint32_t)w * kPair;
    uint8_t* wW = s_w + (uint32_t)w * Dma<GS>::kBytes;
    const TileRef tr = pb.tile(wg, 0);
    const int kb0 = w * GS;
    const int64_t rb = (int64_t)nsb * 144;

    // Activation pieces of rows r0, r0 + 1 (rows >= M read as zero).
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, (uint32_t)((int64_t)pb.M * K * 2));
    auto load_pair = [&](int r0, uint4(&xv)[XI]) {
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int q = lane + 64 * i;
            const int m = q >= XP ? 1 : 0, p = q - m * XP;
            const uint32_t off = q < 2 * XP ? 2u * (uint32_t)((r0 + m) * K + kb0 * QK_K) + 16u * (uint32_t)p : kOOB;
            xv[i] = buf_load16(xr, off);
        }
    };
    // Stage a pair as operand entries at dst and keep the sub-block sums (the four pieces of
    // a sub-block are the four lanes of a quad, which all end with the sum).
    auto stage_pair = [&](const uint4(&xv)[XI], uint8_t* dst, float(&sums)[XI]) {
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int q = lane + 64 * i;
            const int m = q >= XP ? 1 : 0, p = q - m * XP;
            const uint32_t ones = 0x3F803F80u;
            float sm = 0.f;
            sm = dot2(xv[i].x, ones, sm);
            sm = dot2(xv[i].y, ones, sm);
            sm = dot2(xv[i].z, ones, sm);
            sm = dot2(xv[i].w, ones, sm);
            sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
            sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x4E, 0xF, 0xF, false));
            sums[i] = sm;
            if (q < 2 * XP) {
                const int bb = p >> 5, gg = (p >> 3) & 3, t = p & 7;
                *(u32x4_t*)(dst + 16u * (uint32_t)(((bb * 8 + t) * 4 + gg) * 2 + m)) = act_perm(xv[i]);
            }
        }
    };

    // 1. the activations, then the weights; rows 0, 1 are staged while the weights are in
    // flight
    uint4 xa[XI], xb[XI];
    float sa[XI], sb[XI];
    load_pair(0, xa);
    if (MR > 2) load_pair(2, xb);   // rows >= M read as zero
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(tr.base, (uint32_t)(tr.nvalid * rb));
    dma_group<GS, Prob::kPolicy>(wr, wW, rb, kb0, lane);
    __builtin_amdgcn_sched_barrier(0);
    stage_pair(xa, wA, sa);

    // 2. the weights into registers (the compiler waits for the copies into s_w), then rows
    // 2, 3 over the slice -- or, for a two-tile problem, the second tile's weights
    const int n = lane & 15, g = lane >> 4;
    Raw R[GS];
    const uint32_t rrow = (uint32_t)n * (144u * GS);
    auto read_slice = [&]() {
#pragma unroll
        for (int b = 0; b < GS; ++b) {
            const uint8_t* p = wW + rrow + 144u * b;
            R[b].h = *(const uint4*)p;
            R[b].q0 = *(const uint4*)(p + 16 + 32 * g);
            R[b].q1 = *(const uint4*)(p + 32 + 32 * g);
        }
    };
    auto copy_tile = [&](int k) {   // once the slice has been read: tile k into it
        regs_consumed(R);
        const TileRef tk = pb.tile(wg, k);
        dma_group<GS, Prob::kPolicy>(buf_rsrc(tk.base, (uint32_t)(tk.nvalid * rb)), wW, rb, kb0, lane);
    };
    read_slice();
    if constexpr (NT > 1) copy_tile(1);
    if (MR > 2 && rows > 2) stage_pair(xb, wW, sb);

    // 3. the blocks
    u32x4_t A[4];   // block-diagonal operands of four MFMAs: off-diagonal lanes stay zero
#pragma unroll
    for (int t = 0; t < 4; ++t) A[t] = u32x4_t{0u, 0u, 0u, 0u};
    const HdrSel hs = hdr_sel(g);
    const CodeK ck = code_k();
    const int md = (n - 4 * g) & 3;   // the diagonal lanes' activation row
    const uint32_t abase = lds_addr((md < 2 ? wA : wW) + 16u * (uint32_t)(g * 2 + (md & 1)));
    const uint64_t mask = ((1ull << rows) - 1) * 0x1000010000100001ull;   // diag_mask(rows)
    float bt[NT][GS];   // block terms: lane 16i + n holds row n, activation row i
#pragma unroll
    for (int tile = 0; tile < NT; ++tile) {
    if (tile > 0) {   // this tile's weights (the compiler waits for the copies), then the next tile's copy
        __builtin_amdgcn_sched_barrier(0);
        read_slice();
        if (tile + 1 < NT) copy_tile(tile + 1);
    }
#pragma unroll
    for (int b = 0; b < GS; ++b) {
        // lane 16g + n: sums of sub-blocks 2g (lo), 2g + 1 (hi) of block b, rows m: piece
        // (m & 1) * XP + 32b + 8g + 4h of its pair, in staging register ((m & 1) * XP + 32b)
        // / 64 for all g (a 32-aligned run of 32 pieces never straddles 64)
        float lo[MR], hi[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const int q0 = (m & 1) * XP + 32 * b;
            const float src = m < 2 ? sa[q0 / 64] : sb[q0 / 64];
            lo[m] = __shfl(src, (q0 & 63) + 8 * g, 64);
            hi[m] = __shfl(src, (q0 & 63) + 8 * g + 4, 64);
        }
        f32x4_t dlo = {0.f, 0.f, 0.f, 0.f}, dhi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            dlo[m] = -kCodeBiasF * lo[m];
            dhi[m] = -kCodeBiasF * hi[m];
        }
        const uint32_t qd[8] = {R[b].q0.x, R[b].q0.y, R[b].q0.z, R[b].q0.w, R[b].q1.x, R[b].q1.y, R[b].q1.z, R[b].q1.w};
        // low nibbles against operands t = 0..3, then high nibbles against t = 4..7
        a_reads2h(A, abase + (uint32_t)b * 1024u, mask);
#pragma unroll
        for (int t = 0; t < 4; ++t) dlo = mfma(A[t], codes_lo(qd[2 * t], qd[2 * t + 1], ck), dlo);
        a_reads2h(A, abase + (uint32_t)b * 1024u + 512u, mask);
#pragma unroll
        for (int t = 0; t < 4; ++t) dhi = mfma(A[t], codes_hi(qd[2 * t], qd[2 * t + 1], ck), dhi);
        const Hdr H = hdr_decode(R[b].h, hs);
        float t[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) t[m] = block_term(H, dlo[m], dhi[m], lo[m], hi[m]);
        if constexpr (MR == 4) bt[tile][b] = block_sum4(t[0], t[1], t[2], t[3]);
        else bt[tile][b] = block_sum2(t[0], t[1]);
    }
    }

    // 4. the wave's block terms into its slice ([row][column][block], column 2 * tile + m of
    // the four per row), then each output in the fast-mode order over all K parts
    {
        const int i = lane >> 4;   // activation row (MR = 2: rows 0, 1 twice)
        if (i < MR) {
            float* te = (float*)(wW + kRed) + kCols * GS * n;
#pragma unroll
            for (int k = 0; k < NT; ++k)
#pragma unroll
                for (int b = 0; b < GS; ++b) te[(2 * k + i) * GS + b] = bt[k][b];
        }
    }
    __syncthreads();
    // eight lanes per output (uniform trip count: every lane takes part in the cross-lane adds)
    const int per = (int)(blockDim.x >> 3);
    for (int o0 = 0; o0 < kTR * kSmallMaxRows; o0 += per) {
        const int o = o0 + (tid >> 3), rn = (o >> 2) & (kTR - 1), r = o & 3;
        const bool valid = o < kTR * kSmallMaxRows && r < rows;
        auto term = [&](int c, int b) {
            const int k = b / GS;   // the K part (wave) holding block b
            return ((const float*)(s_w + (uint32_t)k * Dma<GS>::kBytes + kRed))[(kCols * rn + c) * GS + (b - k * GS)];
        };
        if constexpr (NT > 1) {
            float v[NT];
#pragma unroll
            for (int k = 0; k < NT; ++k) v[k] = canon_sum8(nsb, lane & 7, [&](int b) { return term(2 * k + r, b); });
            if (valid && (lane & 7) == 0) pb.store_tiles(wg, rn, r, v);
        } else {
            const float v = canon_sum8(nsb, lane & 7, [&](int b) { return term(r, b); });
            if (valid && (lane & 7) == 0) pb.store(wg, rn, r, v);
        }
    }
}

template <int MR, class Prob>
hipError_t run_gemvm(const Prob& pb, int nsb, unsigned nwg, const uint16_t* x, int K, hipStream_t st) {
    // KP waves of BPK blocks: the largest KP <= 8 that divides nsb with a supported BPK
    for (int kp = kMaxW; kp >= 1; --kp) {
        if (nsb % kp || 64 * kp < kTR * MR) continue;   // the final reduction uses kTR * MR threads
        const int bpk = nsb / kp;
        const dim3 grid(nwg), block(64 * kp);
#define AIPU_LM(B)                                                                       \
    case B: hipLaunchKernelGGL((k_gemvm<MR, B, Prob>), grid, block, 0, st, pb, x, K); return hipGetLastError();
        switch (bpk) {
            AIPU_LM(1)
            AIPU_LM(2)
            AIPU_LM(3)
            AIPU_LM(4)
            default: break;
        }
#undef AIPU_LM
    }
    return hipErrorNotSupported;
}

// ------------------------------------------------------------------ planning
int pick_pd(int bpk) {
    for (int pd = 4; pd >= 2; --pd)
        if (bpk % pd == 0) return pd;
    return 1;
}

// T tiles per workgroup, nact staged activations of MR rows.  Returns false when the shape
// does not fit the kernel's staging or LDS limits.
bool make_plan(int nsb, int T, int nact, int MR, int kp_max, Plan& p) {
    int best = 0;
    for (int kp = 1; kp <= kp_max && kp * T <= kMaxW; ++kp)
        if (nsb % kp == 0) best = kp;
    if (best == 0) return false;
    p.KP = best;
    p.bpk = nsb / best;
    p.PD = pick_pd(p.bpk);
    p.W = T * best;
    p.nact = nact;
    const int64_t ent = 8LL * 4 * MR;
    p.lds = ent * 16 + (int64_t)nact * nsb * (ent * 16 + 8LL * MR * 4) + (int64_t)p.W * kTR * MR * 4;
    const int64_t pieces = (int64_t)nact * MR * nsb * 32;
    return p.lds <= kMaxLds && pieces <= (int64_t)kXL * 64 * p.W;
}

template <int MR, class Prob>
hipError_t run_mfma(const Prob& pb, const Plan& pl, unsigned nwg, const uint16_t* X, int64_t xstride,
                    int64_t xbytes, int K, int M, hipStream_t st) {
    const dim3 grid(nwg), block(64 * pl.W);
    const size_t lds = (size_t)pl.lds;
#define AIPU_LAUNCH(PDV)                                                                                         \
    hipLaunchKernelGGL((k_mfma_gemv<MR, PDV, Prob>), grid, block, lds, st, pb, X, xstride, (uint32_t)xbytes, K, M, \
                       pl.nact, pl.KP, pl.bpk)
    switch (pl.PD) {
        case 1: AIPU_LAUNCH(1); break;
        case 2: AIPU_LAUNCH(2); break;
        case 3: AIPU_LAUNCH(3); break;
        default: AIPU_LAUNCH(4); break;
    }
#undef AIPU_LAUNCH
    return hipGetLastError();
}

// Single-row plan: T tiles per workgroup, each split into KP parts of BPK = GS * NG blocks.
struct Plan1 {
    int KP, GS, NG, XI, W;
    int64_t lds;   // dynamic LDS (the weight slices)
};

constexpr int64_t kMaxLds1 = 80 * 1024;   // two workgroups per CU

int dma_bytes(int gs) { return ((16 * 9 * gs + 63) / 64) * 1024; }
// static LDS of k_gemv1<GS, XI>: activation slices (one per wave, or one per K part when the
// tiles of a workgroup share them), reduction
int64_t static_lds1(int xi, bool share) {
    return (int64_t)(share ? kMaxW / 2 : kMaxW) * 2 * xi * 544 + kMaxW * kTR * 4;
}

// canon: the plain GEMV's block-term buffer (16 rows x 8 waves x 2 XI blocks) is static LDS too
bool make_plan1(int nsb, int T, int kp_max, Plan1& p, bool share = false, bool canon = false) {
    for (int kp = (kp_max < kMaxW / T ? kp_max : kMaxW / T); kp >= 1; --kp) {
        if (nsb % kp) continue;
        const int bpk = nsb / kp;
        const int xi_need = (bpk * 32 + 63) / 64;
        const int xi = xi_need <= 2 ? 2 : (xi_need <= 4 ? 4 : (xi_need <= 8 ? 8 : 0));
        if (xi == 0) continue;
        for (int gs = 3; gs >= 1; --gs) {
            if (bpk % gs) continue;
            const int W = T * kp;
            const int64_t lds = (int64_t)W * dma_bytes(gs);
            const int64_t bterm = canon ? (int64_t)kTR * kMaxW * 2 * xi * 4 : 0;
            if (lds + static_lds1(xi, share) + bterm > kMaxLds1) continue;
            p = Plan1{kp, gs, bpk / gs, xi, W, lds};
            return true;
        }
    }
    return false;
}

template <class Prob>
hipError_t run1(const Prob& pb, const Plan1& pl, unsigned nwg, const uint16_t* X, int64_t xstride, int64_t xbytes,
                int K, hipStream_t st, int tpw = 1) {
    const dim3 grid(nwg), block(64 * pl.W);
    const size_t lds = (size_t)pl.lds;
#define AIPU_L1(GSV, XIV)                                                                                      \
    if (tpw > 1)                                                                                               \
        hipLaunchKernelGGL((k_gemv1<GSV, XIV, Prob, true>), grid, block, lds, st, pb, X, xstride, (uint32_t)xbytes, \
                           K, pl.KP, pl.NG, tpw);                                                              \
    else                                                                                                       \
        hipLaunchKernelGGL((k_gemv1<GSV, XIV, Prob, false>), grid, block, lds, st, pb, X, xstride,               \
                           (uint32_t)xbytes, K, pl.KP, pl.NG, 1)
#define AIPU_L1X(GSV)                        \
    switch (pl.XI) {                         \
        case 2: AIPU_L1(GSV, 2); break;      \
        case 4: AIPU_L1(GSV, 4); break;      \
        default: AIPU_L1(GSV, 8); break;     \
    }
    switch (pl.GS) {
        case 1: AIPU_L1X(1); break;
        case 2: AIPU_L1X(2); break;
        default: AIPU_L1X(3); break;
    }
#undef AIPU_L1X
#undef AIPU_L1
    return hipGetLastError();
}

// Small-batch plan: KP <= 8 waves of GS <= 3 blocks (three blocks' weights, one block's
// operands and four rows' sums fill the 128 registers of four waves per SIMD), the weight
// slices and staged pair within half the CU's LDS.
struct PlanS {
    int KP, GS;
    int64_t lds;   // dynamic LDS (the weight slices)
};

bool make_plans(int nsb, PlanS& p) {
    for (int kp = kMaxW; kp >= 1; --kp) {
        if (nsb % kp || nsb / kp > 3) continue;
        const int gs = nsb / kp;
        const int64_t lds = (int64_t)kp * dma_bytes(gs);
        if (lds + (int64_t)kMaxW * gs * 1024 > kMaxLds1) continue;
        p = PlanS{kp, gs, lds};
        return true;
    }
    return false;
}

template <int MR, class Prob>
hipError_t runs_mr(const Prob& pb, const PlanS& pl, unsigned nwg, const uint16_t* X, int K, hipStream_t st) {
    const dim3 grid(nwg), block(64 * pl.KP);
    const size_t lds = (size_t)pl.lds;
    switch (pl.GS) {
        case 1: hipLaunchKernelGGL((k_gemvs<1, kMaxW, MR, Prob>), grid, block, lds, st, pb, X, K); break;
        case 2: hipLaunchKernelGGL((k_gemvs<2, kMaxW, MR, Prob>), grid, block, lds, st, pb, X, K); break;
        default: hipLaunchKernelGGL((k_gemvs<3, kMaxW, MR, Prob>), grid, block, lds, st, pb, X, K); break;
    }
    return hipGetLastError();
}

hipError_t runs(const ProbPlain<4>& pb, const PlanS& pl, unsigned nwg, const uint16_t* X, int K, hipStream_t st) {
    return pb.M <= 2 ? runs_mr<2>(pb, pl, nwg, X, K, st) : runs_mr<4>(pb, pl, nwg, X, K, st);
}

// Shapes the small-batch kernel covers: K / 256 split into at most 8 parts of 1 .. 4 blocks,
// with enough waves for the reduction of mr rows.
bool gemvm_supported(int nsb, int mr) {
    for (int kp = kMaxW; kp >= 1; --kp)
        if (nsb % kp == 0 && nsb / kp <= 4 && 64 * kp >= kTR * mr) return true;
    return false;
}

// One-row shapes where the 16-row-tile kernel (k_gemv1) measured faster than the persistent one
// (MI355X, a HIP graph of launches over weights rotated through 0.6 GB, N = 2048..16384 against
// K = 2048..8192): every CU gets one or two 16-row tiles and K <= 4096 (C0, 4096 x 4096: 4.41
// against 4.68 us); or at least one tile per CU and K = 2048 (the persistent kernel's second copy
// round is 128 B per row; 16384 x 2048: 6.83 against 9.21 us) or K > 6144 (two block pairs per
// persistent compute wave; 4096 x 8192: 5.97 against 7.94 us).  Both kernels form a row in the
// same order, so the choice never changes a result bit.
bool prefer_gemv1(int64_t N, int64_t K) {
    const int64_t t16 = (N + kTR - 1) / kTR, cus = device_cu_count();
    if (t16 < cus) return false;
    if (K == 2048 || K > 6144) return true;
    return K <= 4096 && t16 <= 2 * cus;
}

template <int MR>
hipError_t plain_pass(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, int M, uint16_t* y, float* yf,
                      int64_t ystride, hipStream_t st) {
    const int nsb = (int)(K / QK_K);
    const ProbPlain<MR> pb{W, N, row_bytes(T_Q4_K, K), y, yf, ystride, M};
    const unsigned nwg = (unsigned)((N + kTR - 1) / kTR);
    if constexpr (MR == 1) {
        Plan1 p1;
        const bool k1 = make_plan1(nsb, 1, kMaxW, p1, false, true);
        if (gemv_persist_supported(N, K) && !(k1 && prefer_gemv1(N, K))) return launch_gemv_persist(W, N, K, x, y, yf, st);
        if (k1) return run1(pb, p1, nwg, x, 0, (int64_t)K * 2, (int)K, st);
    } else {
        if (gemvm_supported(nsb, MR)) return run_gemvm<MR>(pb, nsb, nwg, x, (int)K, st);
    }
    Plan pl;
    if (!make_plan(nsb, 1, 1, MR, kMaxW, pl)) return hipErrorInvalidValue;
    return run_mfma<MR>(pb, pl, nwg, x, 0, (int64_t)M * K * 2, (int)K, M, st);
}

}  // namespace

// Whether the matrix-core GEMV serves this shape (Q4_K, any M, the staging limits).  Every
// shape of the persistent one-row kernel is served (K <= 8192, block counts such as 17, 19,
// 23, 29 and 31 included, which no k_mfma_gemv plan splits): a row without a multi-row kernel
// in that order runs as its own one-row launch, so the rows of a batch keep their one-row bits.
bool gemv_mfma_supported(int64_t N, int64_t K, int64_t M) {
    if (N < 1 || K < QK_K || K % QK_K != 0 || M < 1) return false;
    if (N * row_bytes(T_Q4_K, K) >= (int64_t)1 << 40) return false;
    if (gemv_persist_supported(N, K)) return true;
    Plan pl;
    const int mr = M >= 4 ? 4 : (M >= 2 ? 2 : 1);
    return K <= (1 << 20) && make_plan((int)(K / QK_K), 1, 1, mr, kMaxW, pl);
}

// y[M][N] (row stride ystride) = x[M][K] . W^T, in passes of at most 8 activation rows.
// A pass goes to a multi-row kernel only if that kernel forms each row exactly as the one-row
// launch does (two rows on the persistent one-row kernel itself, the persistent row-pair
// kernel, k_gemvm, k_gemvs: the order of mfma_gemv.hpp,
// which the single-row kernels k_gemv1p and k_gemv1 follow); every other row runs as its own
// one-row launch, so each row of the result is bit-identical to the one-row call on that row
// at every shape.  `dense` swaps the persistent row-pair kernel for the dense one (rows within
// the tolerance of their one-row results); nothing else changes.
hipError_t launch_gemv_mfma(const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                            float* y_f32, int64_t ystride, hipStream_t st, bool dense) {
    const uint8_t* W = (const uint8_t*)w;
    const int nsb = (int)(K / QK_K);
    PlanS ps;
    const bool small = make_plans(nsb, ps);
    Plan1 p1;
    const bool canon1 = gemv_persist_supported(N, K) || make_plan1(nsb, 1, kMaxW, p1, false, true);   // one-row launch in that order
    for (int64_t m0 = 0; m0 < M;) {
        const int left = (int)(M - m0 < 8 ? M - m0 : 8);
        const uint16_t* xm = x + m0 * K;
        uint16_t* ym = y + m0 * ystride;
        float* yfm = y_f32 ? y_f32 + m0 * ystride : nullptr;
        if (left >= 2 && canon1) {
            if (left == 2 && !dense && gemv_persist2_supported(N, K)) {   // two rows on the one-row kernel
                const hipError_t e = launch_gemv_persist2(W, N, K, xm, ym, yfm, ystride, st);
                if (e != hipSuccess) return e;
                m0 += 2;
                continue;
            }
            if (gemv_persist_m_supported(N, K, left, dense)) {   // two to eight rows, one persistent pass
                const hipError_t e = launch_gemv_persist_m(W, N, K, xm, left, ym, yfm, ystride, dense, st);
                if (e != hipSuccess) return e;
                m0 += left;
                continue;
            }
            if (left >= 5 && gemvm_supported(nsb, 8)) {   // five to eight rows in one pass
                const ProbPlain<8> pb{W, N, row_bytes(T_Q4_K, K), ym, yfm, ystride, left};
                const hipError_t e = run_gemvm<8>(pb, nsb, (unsigned)((N + kTR - 1) / kTR), xm, (int)K, st);
                if (e != hipSuccess) return e;
                m0 += left;
                continue;
            }
            if (small) {   // two to four rows, the weights read once
                const int mr = left < kSmallMaxRows ? left : kSmallMaxRows;
                const ProbPlain<4> pb{W, N, row_bytes(T_Q4_K, K), ym, yfm, ystride, mr};
                const hipError_t e = runs(pb, ps, (unsigned)((N + kTR - 1) / kTR), xm, (int)K, st);
                if (e != hipSuccess) return e;
                m0 += mr;
                continue;
            }
            if (gemv_persist2_supported(N, K)) {   // no other multi-row kernel: two rows at a time
                const hipError_t e = launch_gemv_persist2(W, N, K, xm, ym, yfm, ystride, st);
                if (e != hipSuccess) return e;
                m0 += 2;
                continue;
            }
        }
        const hipError_t e = plain_pass<1>(W, N, K, xm, 1, ym, yfm, ystride, st);
        if (e != hipSuccess) return e;
        ++m0;
    }
    return hipSuccess;
}

// Threads per gate/up workgroup of the plan launch_moe_gateup_mfma picks for an
// H / 256 = nsb block row when it routes in the kernel (0: no plan); in-kernel routing ranks
// one key per thread, so this bounds E.
static int gateup_route_threads(int nsb, int64_t E) {
    const int need = (int)((E + 7) & ~7);
    Plan1 p1;
    if (make_plan1(nsb, 2, 4, p1, true) && p1.W * 64 >= need) return p1.W * 64;
    Plan pl;
    if (make_plan(nsb, 2, 1, 1, 4, pl)) return pl.W * 64;
    return 0;
}

bool moe_route_in_kernel(int64_t E, int topk, int64_t H) {
    if (!(E >= 1 && E <= kRouteMaxE && topk >= 1 && topk <= kRouteMaxTopk && topk <= E)) return false;
    if (H < QK_K || H % QK_K) return false;
    return gateup_route_threads((int)(H / QK_K), E) >= (int)((E + 7) & ~7);
}

hipError_t launch_moe_gateup_mfma(const uint8_t* G, const uint8_t* U, const uint8_t* shG, const uint8_t* shU,
                                  const MoeRoute& route, int topk, int nslots, int64_t E, int64_t H, int64_t I,
                                  const uint16_t* x, uint16_t* h, hipStream_t st) {
    const int nsb = (int)(H / QK_K);
    if (I % kTR != 0) return hipErrorInvalidValue;
    if (route.logits && !moe_route_in_kernel(E, topk, H)) return hipErrorInvalidValue;
    const int64_t rb = row_bytes(T_Q4_K, H);
    const ProbGateUp pb{G, U, shG, shU, route, topk, (int)E, (int)(I / kTR), rb, rb * I, h, I, 0};
    const int itiles = (int)(I / kTR);
    const int64_t ntiles = (int64_t)nslots * itiles;
    // tiles of one slot per workgroup: the count that takes the fewest tile-times at two
    // workgroups per CU (ties to the larger count: fewer routing and staging passes)
    const int64_t wave_slots = 2LL * device_cu_count();
    int tpw = 1;
    int64_t best = (ntiles + wave_slots - 1) / wave_slots;
    for (int c = 2; c <= 4; c *= 2) {
        if (itiles % c) continue;
        const int64_t cost = (ntiles / c + wave_slots - 1) / wave_slots * c;
        if (cost <= best) {
            best = cost;
            tpw = c;
        }
    }
    const unsigned nwg = (unsigned)(ntiles / tpw);
    Plan1 p1;
    if (make_plan1(nsb, 2, 4, p1, true) && p1.W * 64 >= (route.logits ? (int)((E + 7) & ~7) : 0))
        return run1(pb, p1, nwg, x, 0, H * 2, (int)H, st, tpw);
    Plan pl;
    if (!make_plan(nsb, 2, 1, 1, 4, pl) || pl.W * 64 < (route.logits ? (int)((E + 7) & ~7) : 0)) return hipErrorInvalidValue;
    return run_mfma<1>(pb, pl, (unsigned)ntiles, x, 0, H * 2, (int)H, 1, st);   // one tile per workgroup
}

// One down launch over `nslots` slots (at most one workgroup's waves).
static hipError_t down_once(const ProbDown& pb, int64_t I, const uint16_t* h, hipStream_t st) {
    const int nsb = (int)(I / QK_K);
    const unsigned nwg = (unsigned)((pb.H + kTR - 1) / kTR);
    const int kpmax = kMaxW / pb.nslots > 0 ? kMaxW / pb.nslots : 1;
    Plan1 p1;
    if (pb.nslots <= kMaxW && make_plan1(nsb, pb.nslots, kpmax, p1))
        return run1(pb, p1, nwg, h, I, (int64_t)pb.nslots * I * 2, (int)I, st);
    Plan pl;
    if (!make_plan(nsb, pb.nslots, pb.nslots, 1, kpmax, pl)) return hipErrorInvalidValue;
    return run_mfma<1>(pb, pl, nwg, h, I, (int64_t)pb.nslots * I * 2, (int)I, 1, st);
}

hipError_t launch_moe_down_mfma(const uint8_t* D, const uint8_t* shD, const int32_t* sel, const uint16_t* selw,
                                int topk, int nslots, int64_t E, int64_t H, int64_t I, const uint16_t* h, uint16_t* y,
                                int passthrough, hipStream_t st, float* acc_scratch, const uint16_t* resid) {
    const int64_t rb = row_bytes(T_Q4_K, I);
    if (nslots <= kMaxW) {
        ProbDown pb{D, shD, sel, selw, topk, nslots, (int)E, passthrough, H, rb, rb * H, y};
        pb.resid = resid;
        return down_once(pb, I, h, st);
    }
    // topk routed slots + the shared slot: routed slots first (fp32 running sum kept), then
    // the shared slot continues the same sum and rounds.
    if (nslots != topk + 1 || topk > kMaxW || !acc_scratch || passthrough) return hipErrorInvalidValue;
    ProbDown routed{D, shD, sel, selw, topk, topk, (int)E, 0, H, rb, rb * H, y};
    routed.acc_out = acc_scratch;
    hipError_t e = down_once(routed, I, h, st);
    if (e != hipSuccess) return e;
    ProbDown shared{D, shD, sel, selw, 0, 1, (int)E, 0, H, rb, rb * H, y};
    shared.acc_in = acc_scratch;
    shared.resid = resid;
    return down_once(shared, I, h + (int64_t)topk * I, st);
}

// ------------------------------------------- batched MoE over the expert union (M = 2..8)
// Slot u of the union holds expert uidx[u] (-1 = the shared expert); *nslots of the grid's
// slots are live, the rest of the workgroups return at once.  Gate/up: workgroup
// ((u * 2 + part) * itiles + it) computes rows it*16.. of the gate (part 0) or up (part 1)
// projection of slot u for all M rows -> gu[u][part][m][i].  Down: workgroup (u * htiles +
// it) computes output rows it*16.. of slot u against h[u][m][:] -> y[u][m][d].
template <int MR>
struct ProbUGateUp {
    const uint8_t *G, *U, *shG, *shU;
    const int32_t* uidx;
    const int32_t* nslots;
    int itiles, M;
    int64_t rb, ebytes, I;
    uint16_t* gu;
    static constexpr bool kRoutes = false;
    static constexpr bool kShareAct = false;
    static constexpr uint32_t kPolicy = kNT;   // streaming (default caching measured slower here)
    static constexpr int kTiles = 1;
    __device__ void setup(int, uint32_t*, uint32_t*, int32_t*, uint16_t*) {}
    __device__ bool active(int wg) const { return wg / (2 * itiles) < *nslots; }
    __device__ const uint16_t* act(int, const uint16_t* X) const { return X; }
    __device__ TileRef tile(int wg, int) const {
        const int u = wg / (2 * itiles), part = (wg / itiles) & 1, it = wg % itiles;
        const int e = __builtin_amdgcn_readfirstlane(uidx[u]);
        const uint8_t* base = e < 0 ? (part ? shU : shG) : (part ? U : G) + (int64_t)e * ebytes;
        return TileRef{base + (int64_t)it * kTR * rb, kTR, 0};
    }
    __device__ void store(int wg, int n, int r, float v) const {
        if (r >= M) return;
        const int u = wg / (2 * itiles), part = (wg / itiles) & 1, it = wg % itiles;
        gu[(((int64_t)u * 2 + part) * M + r) * I + (int64_t)it * kTR + n] = (uint16_t)bf16_rne(v);
    }
};

template <int MR>
struct ProbUDown {
    const uint8_t *D, *shD;
    const int32_t* uidx;
    const int32_t* nslots;
    int htiles, M;
    int64_t rb, ebytes, I, H;
    const uint16_t* h;
    uint16_t* y;
    static constexpr bool kRoutes = false;
    static constexpr bool kShareAct = false;
    static constexpr uint32_t kPolicy = kNT;   // streaming (default caching measured slower here)
    static constexpr int kTiles = 1;
    __device__ void setup(int, uint32_t*, uint32_t*, int32_t*, uint16_t*) {}
    __device__ bool active(int wg) const { return wg / htiles < *nslots; }
    __device__ const uint16_t* act(int wg, const uint16_t*) const { return h + (int64_t)(wg / htiles) * M * I; }
    __device__ TileRef tile(int wg, int) const {
        const int u = wg / htiles, it = wg % htiles;
        const int e = __builtin_amdgcn_readfirstlane(uidx[u]);
        const uint8_t* base = e < 0 ? shD : D + (int64_t)e * ebytes;
        const int64_t nv = H - (int64_t)it * kTR;
        return TileRef{base + (int64_t)it * kTR * rb, (int)(nv < kTR ? nv : kTR), 0};
    }
    __device__ void store(int wg, int n, int r, float v) const {
        const int u = wg / htiles, it = wg % htiles;
        const int64_t d = (int64_t)it * kTR + n;
        if (r >= M || d >= H) return;
        y[((int64_t)u * M + r) * H + d] = (uint16_t)bf16_rne(v);
    }
};

// The down leg of a two-row pass: workgroup (u * htilesT + it) computes tiles NT it .. NT it +
// NT - 1 of slot u (each copied while the one before computes), each exactly as ProbUDown<2>
// would.
template <int NT>
struct ProbUDownT {
    const uint8_t *D, *shD;
    const int32_t* uidx;
    const int32_t* nslots;
    int htilesT, M;
    int64_t rb, ebytes, I, H;
    const uint16_t* h;
    uint16_t* y;
    static constexpr uint32_t kPolicy = kNT;
    static constexpr int kTiles = NT;
    __device__ bool active(int wg) const { return wg / htilesT < *nslots; }
    __device__ const uint16_t* act(int wg, const uint16_t*) const { return h + (int64_t)(wg / htilesT) * M * I; }
    __device__ TileRef tile(int wg, int part) const {
        const int u = wg / htilesT, it = NT * (wg % htilesT) + part;
        const int e = __builtin_amdgcn_readfirstlane(uidx[u]);
        const uint8_t* base = e < 0 ? shD : D + (int64_t)e * ebytes;
        const int64_t nv = H - (int64_t)it * kTR;   // a tile past H reads as zero
        return TileRef{base + (nv > 0 ? (int64_t)it * kTR * rb : 0), (int)(nv <= 0 ? 0 : nv < kTR ? nv : kTR), 0};
    }
    __device__ void store_tiles(int wg, int n, int r, const float (&v)[NT]) const {
        if (r >= M) return;
        const int u = wg / htilesT;
        uint16_t* yr = y + ((int64_t)u * M + r) * H;
#pragma unroll
        for (int k = 0; k < NT; ++k) {
            const int64_t d = (int64_t)(NT * (wg % htilesT) + k) * kTR + n;
            if (d < H) yr[d] = (uint16_t)bf16_rne(v[k]);
        }
    }
};
constexpr int kDownTiles = 4;

// Gate/up with the SwiGLU fused, for the small-batch kernel: workgroup (u * itiles + it)
// computes rows it*16.. of both the gate and the up projection of slot u (two tiles, the
// second copied while the first computes) and writes h[u][m][i] = bf16(silu(g) * u) -- the
// same rounding steps as the separate pass.
struct ProbUGateUpH {
    const uint8_t *G, *U, *shG, *shU;
    const int32_t* uidx;
    const int32_t* nslots;
    int itiles, M;
    int64_t rb, ebytes, I;
    uint16_t* h;
    static constexpr uint32_t kPolicy = kNT;   // streaming (default caching measured slower here)
    static constexpr int kTiles = 2;
    __device__ bool active(int wg) const { return wg / itiles < *nslots; }
    __device__ const uint16_t* act(int, const uint16_t* X) const { return X; }
    __device__ TileRef tile(int wg, int part) const {
        const int u = wg / itiles, it = wg % itiles;
        const int e = __builtin_amdgcn_readfirstlane(uidx[u]);
        const uint8_t* base = e < 0 ? (part ? shU : shG) : (part ? U : G) + (int64_t)e * ebytes;
        return TileRef{base + (int64_t)it * kTR * rb, kTR, 0};
    }
    __device__ void store_tiles(int wg, int n, int r, const float (&v)[2]) const {
        if (r >= M) return;
        const float g = v[0];
        const int u = wg / itiles, it = wg % itiles;
        const uint32_t gb = bf16_rne(g), ub = bf16_rne(v[1]);
        h[((int64_t)u * M + r) * I + (int64_t)it * kTR + n] =
            (uint16_t)bf16_rne(bf16_to_f32(glm_silu_bf16(gb)) * bf16_to_f32(ub));
    }
};

bool moe_union_supported(int64_t H, int64_t I, int M) {
    const int mr = M <= 2 ? 2 : (M <= 4 ? 4 : 8);
    return M >= 1 && M <= 8 && I % kTR == 0 && gemvm_supported((int)(H / QK_K), mr) &&
           gemvm_supported((int)(I / QK_K), mr);
}

// The union legs: up to four rows on the small-batch kernel (weights copied to LDS) when
// both K's fit its plan, otherwise the register-weight kernel.
template <int MR, class Prob>
static hipError_t union_leg(const Prob& pb, int nsb, unsigned nwg, const uint16_t* x, int K, hipStream_t st) {
    if constexpr (MR <= 4) {
        PlanS ps;
        if (make_plans(nsb, ps)) return pb.M <= 2 ? runs_mr<2>(pb, ps, nwg, x, K, st) : runs_mr<4>(pb, ps, nwg, x, K, st);
    }
    return run_gemvm<MR>(pb, nsb, nwg, x, K, st);
}

template <int MR>
static hipError_t union_gemvs(const MoeUnionArgs& a, hipStream_t st) {
    const int64_t rbH = row_bytes(T_Q4_K, a.H), rbI = row_bytes(T_Q4_K, a.I);
    const int itiles = (int)(a.I / kTR), htiles = (int)((a.H + kTR - 1) / kTR);
    hipError_t e;
    PlanS ps, psI;
    if (MR == 2 && make_plans((int)(a.H / QK_K), ps) && make_plans((int)(a.I / QK_K), psI)) {
        // two rows: gate and up of a tile in one workgroup, h written directly
        const ProbUGateUpH ph{a.G, a.U, a.shG, a.shU, a.uidx, a.nslots, itiles, a.M, rbH, rbH * a.I, a.I, a.h};
        e = runs_mr<2>(ph, ps, (unsigned)(a.max_slots * itiles), a.x, (int)a.H, st);
    } else {
        const ProbUGateUp<MR> pg{a.G, a.U, a.shG, a.shU, a.uidx, a.nslots, itiles, a.M, rbH, rbH * a.I, a.I, a.gu};
        e = union_leg<MR>(pg, (int)(a.H / QK_K), (unsigned)(a.max_slots * 2 * itiles), a.x, (int)a.H, st);
        if (e == hipSuccess) e = a.after_gateup(st);
    }
    if (e != hipSuccess) return e;
    if (MR == 2 && make_plans((int)(a.I / QK_K), psI)) {
        // two rows: kDownTiles tiles of the slot per workgroup
        const int htilesT = (htiles + kDownTiles - 1) / kDownTiles;
        const ProbUDownT<kDownTiles> pd{a.D, a.shD, a.uidx, a.nslots, htilesT, a.M, rbI, rbI * a.H, a.I, a.H, a.h, a.y};
        return runs_mr<2>(pd, psI, (unsigned)(a.max_slots * htilesT), a.h, (int)a.I, st);
    }
    const ProbUDown<MR> pd{a.D, a.shD, a.uidx, a.nslots, htiles, a.M, rbI, rbI * a.H, a.I, a.H, a.h, a.y};
    return union_leg<MR>(pd, (int)(a.I / QK_K), (unsigned)(a.max_slots * htiles), a.h, (int)a.I, st);
}

int moe_union_pass_rows(int64_t H, int64_t I) {
    PlanS p;
    return make_plans((int)(H / QK_K), p) && make_plans((int)(I / QK_K), p) ? 2 : 8;
}

hipError_t launch_moe_union_mfma(const MoeUnionArgs& a, hipStream_t st) {
    if (!moe_union_supported(a.H, a.I, a.M)) return hipErrorInvalidValue;
    if (a.M <= 2) return union_gemvs<2>(a, st);
    if (a.M <= 4) return union_gemvs<4>(a, st);
    return union_gemvs<8>(a, st);
}

bool moe_mfma_supported(int nslots, int64_t H, int64_t I) {
    Plan p1, p2;
    if (I % kTR != 0 || !make_plan((int)(H / QK_K), 2, 1, 1, 4, p1)) return false;
    const auto down_ok = [&](int n) {
        return make_plan((int)(I / QK_K), n, n, 1, kMaxW / n > 0 ? kMaxW / n : 1, p2);
    };
    if (nslots <= kMaxW) return down_ok(nslots);
    return nslots == kMaxW + 1 && down_ok(kMaxW) && down_ok(1);
}

}  // namespace aipu
