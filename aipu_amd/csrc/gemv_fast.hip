// Streaming GEMV kernels (tolerance mode) for Q4_K and bf16 weights, and the two MoE
// expert kernels built on the same lane geometry (see q4k_fast.hpp).
//
// Workgroup shape.  A row's K is split into segments of 2048 weights; `segw` waves of a
// workgroup each own one segment (so each lane's activations are loaded once and stay in
// VGPRs), and `rgc` independent row-groups of segw waves share the workgroup.  Each wave
// processes PASSES item pairs per batch (two items per pass, one per half-wave), reduces
// its partial sums across the half-wave, and the per-segment partials are added in fixed
// segment order through LDS, so results are deterministic.
#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"
#include "q4k_fast.hpp"

namespace aipu {

using namespace q4f;

namespace {

constexpr int kMaxWaves = 8;
constexpr int kMaxVals = 16;   // PASSES * MC per wave

struct StreamGeom {
    int nsb;      // 256-weight blocks per row
    int nseg;     // 2048-weight segments per row
    int segw;     // waves per row-group (segments handled in parallel)
    int spw;      // segments per wave
    int rgc;      // row-groups per workgroup
    int nbatch;   // batches per row-group
    int64_t npairs;
};

template <int TYPE>
struct Pass;

// Q4_K: header + 32 B of qs per lane.
template <>
struct Pass<T_Q4_K> {
    typedef Raw R;
    __device__ static R load(const uint8_t* row, int blk, const Geo& G) { return raw_load(row + (int64_t)blk * 144, G); }
    __device__ static void act(Act& A, const uint16_t* xrow, int seg, const Geo& G, bool valid) {
        act_load(A, xrow, seg, G, valid);
    }
    template <int MC>
    __device__ static void part(const R& r, const Act (&A)[MC], float (&out)[MC], const Geo& G) {
        const Hdr H = hdr_decode(r.h, G);
#pragma unroll
        for (int m = 0; m < MC; ++m) {
            float Slo, Shi;
            code_dots(r, A[m], Slo, Shi);
            out[m] = lane_part(H, Slo, Shi, A[m]);
        }
    }
};

// bf16 weights: the lane's 64 consecutive weights, 8 x 16 B.
struct RawBF16 {
    uint4 v[8];
};

template <>
struct Pass<T_BF16> {
    typedef RawBF16 R;
    __device__ static R load(const uint8_t* row, int blk, const Geo& G) {
        const uint4* p = (const uint4*)(row + (int64_t)blk * 512 + 128 * G.g);
        R r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r.v[i] = p[i];
        return r;
    }
    __device__ static void act(Act& A, const uint16_t* xrow, int seg, const Geo& G, bool valid) {
        if (!valid) {
            act_zero(A);
            return;
        }
        const uint4* p = (const uint4*)(xrow + (int64_t)(seg * kSegBlocks + G.bs) * QK_K + 64 * G.g);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 v = p[i];
            A.xa[4 * i + 0] = v.x;
            A.xa[4 * i + 1] = v.y;
            A.xa[4 * i + 2] = v.z;
            A.xa[4 * i + 3] = v.w;
        }
        A.alo = A.ahi = 0.f;
    }
    template <int MC>
    __device__ static void part(const R& r, const Act (&A)[MC], float (&out)[MC], const Geo&) {
#pragma unroll
        for (int m = 0; m < MC; ++m) {
            float s0 = 0.f, s1 = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                s0 = dot2(A[m].xa[4 * i + 0], r.v[i].x, s0);
                s1 = dot2(A[m].xa[4 * i + 1], r.v[i].y, s1);
                s0 = dot2(A[m].xa[4 * i + 2], r.v[i].z, s0);
                s1 = dot2(A[m].xa[4 * i + 3], r.v[i].w, s1);
            }
            out[m] = s0 + s1;
        }
    }
};

template <int N>
struct Pow2 {
    static constexpr int v = N <= 1 ? 1 : N <= 2 ? 2 : N <= 4 ? 4 : N <= 8 ? 8 : N <= 16 ? 16 : 32;
    static constexpr int lg = v == 1 ? 0 : v == 2 ? 1 : v == 4 ? 2 : v == 8 ? 3 : v == 16 ? 4 : 5;
};

// --------------------------------------------------------------------- items
struct PlainItems {
    const uint8_t* W;
    int64_t N, rb;
    __device__ int expert(int64_t) const { return 0; }
    __device__ const uint8_t* row_e(int64_t pair, int half, int) const {
        int64_t r = 2 * pair + half;
        r = r < N ? r : N - 1;
        return W + r * rb;
    }
    __device__ const uint8_t* row(int64_t pair, int half) const { return row_e(pair, half, 0); }
};

struct PlainEpi {
    uint16_t* Y;
    float* Yf;
    int64_t N;
    int mrows;
    __device__ void operator()(int64_t pair, int m, float v0, float v1) const {
        if (m >= mrows) return;
        const int64_t r = 2 * pair;
        if (r < N) {
            Y[m * N + r] = (uint16_t)bf16_rne(v0);
            if (Yf) Yf[m * N + r] = v0;
        }
        if (r + 1 < N) {
            Y[m * N + r + 1] = (uint16_t)bf16_rne(v1);
            if (Yf) Yf[m * N + r + 1] = v1;
        }
    }
};

// MoE gate/up: pair = slot * I + i; half 0 reads gate row i of the slot's expert, half 1
// the up row.  Slot `topk` (if present) is the shared expert.
struct GateUpItems {
    const uint8_t* G;
    const uint8_t* U;
    const uint8_t* shG;
    const uint8_t* shU;
    const int32_t* sel;
    int topk, nslots, I;
    int E;
    int64_t ebytes, rb;
    // Routed expert of the item's slot (loaded from the router's output), clamped to [0, E).
    __device__ int expert(int64_t pair) const {
        const int npairs = nslots * I;
        const int p = (int)(pair < npairs ? pair : npairs - 1);
        const int s = p / I;
        // a buffer load (0 beyond the topk entries) rather than a branch around a load: at
        // a branch join the compiler would wait for every earlier load
        const int e = (int)buf_load4(buf_rsrc(sel, 4u * (uint32_t)topk), 4u * (uint32_t)s);
        return e < 0 ? 0 : (e >= E ? E - 1 : e);
    }
    __device__ const uint8_t* row_e(int64_t pair, int half, int e) const {
        const int npairs = nslots * I;
        const int p = (int)(pair < npairs ? pair : npairs - 1);
        const int s = p / I;
        const int i = p - s * I;
        const uint8_t* routed = (half ? U : G) + (int64_t)e * ebytes;
        const uint8_t* shared = half ? shU : shG;
        return (s < topk ? routed : shared) + (int64_t)i * rb;
    }
    __device__ const uint8_t* row(int64_t pair, int half) const { return row_e(pair, half, expert(pair)); }
};

// h = bf16(f32(glm_silu(bf16 gate)) * f32(bf16 up))  (tools/glm_model_q4k_ref.py:705-707)
struct GateUpEpi {
    uint16_t* h;
    int64_t npairs;
    __device__ void operator()(int64_t pair, int, float v0, float v1) const {
        if (pair >= npairs) return;
        const uint32_t g = bf16_rne(v0), u = bf16_rne(v1);
        h[pair] = (uint16_t)bf16_rne(bf16_to_f32(glm_silu_bf16(g)) * bf16_to_f32(u));
    }
};

// ------------------------------------------------------------ stream kernel
template <int TYPE, int MC, int PASSES, class Items, class Epi>
__global__ __launch_bounds__(kMaxWaves * 64) void k_stream(Items items, Epi epi, const uint16_t* __restrict__ X,
                                                           int64_t K, int mrows, StreamGeom sg) {
    constexpr int NV = PASSES * MC;
    constexpr int VP = Pow2<NV>::v;
    constexpr int LV = Pow2<NV>::lg;
    static_assert(NV <= kMaxVals, "too many values per wave");
    __shared__ float red[2][kMaxWaves][kMaxVals][2];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rg = wave / sg.segw, wseg = wave - rg * sg.segw;
    const Geo G = make_geo(lane);

    Act A[MC];
    if (sg.spw == 1) {
        const int blk = wseg * kSegBlocks + G.bs;
#pragma unroll
        for (int m = 0; m < MC; ++m) Pass<TYPE>::act(A[m], X + (int64_t)m * K, wseg, G, m < mrows && blk < sg.nsb);
    }

    int buf = 0;
    for (int b = 0; b < sg.nbatch; ++b) {
        const int64_t P0 = (((int64_t)blockIdx.x * sg.rgc + rg) * sg.nbatch + b) * PASSES;
        float part[PASSES][MC];
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
#pragma unroll
            for (int m = 0; m < MC; ++m) part[p][m] = 0.f;

        for (int si = 0; si < sg.spw; ++si) {
            const int seg = wseg + si * sg.segw;
            const int blk = seg * kSegBlocks + G.bs;
            const bool bvalid = seg < sg.nseg && blk < sg.nsb;
            if (sg.spw > 1) {
#pragma unroll
                for (int m = 0; m < MC; ++m) Pass<TYPE>::act(A[m], X + (int64_t)m * K, seg, G, m < mrows && bvalid);
            }
            typename Pass<TYPE>::R r[PASSES];
#pragma unroll
            for (int p = 0; p < PASSES; ++p) r[p] = Pass<TYPE>::load(items.row(P0 + p, G.half), bvalid ? blk : 0, G);
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                float o[MC];
                Pass<TYPE>::template part<MC>(r[p], A, o, G);
#pragma unroll
                for (int m = 0; m < MC; ++m) part[p][m] += bvalid ? o[m] : 0.f;
            }
        }

        float v[VP];
#pragma unroll
        for (int i = 0; i < VP; ++i) v[i] = i < NV ? part[i / MC][i % MC] : 0.f;
        const float tot = half_reduce<VP>(v, lane);
        const int vi = (G.s >> (5 - LV)) & (VP - 1);
        if ((G.s & ((32 >> LV) - 1)) == 0 && vi < NV) red[buf][wave][vi][G.half] = tot;
        __syncthreads();
        const int t = threadIdx.x;
        if (t < sg.rgc * NV) {
            const int erg = t / NV, ev = t - erg * NV;
            float v0 = 0.f, v1 = 0.f;
            for (int w = 0; w < sg.segw; ++w) {
                v0 += red[buf][erg * sg.segw + w][ev][0];
                v1 += red[buf][erg * sg.segw + w][ev][1];
            }
            const int64_t pair = (((int64_t)blockIdx.x * sg.rgc + erg) * sg.nbatch + b) * PASSES + ev / MC;
            if (pair < sg.npairs) epi(pair, ev % MC, v0, v1);
        }
        buf ^= 1;
    }
}

// -------------------------------------------------------- row kernel (M = 1)
// For M = 1 and K <= 8192 each wave walks whole row pairs (half-wave = one row, all
// segments), so no cross-wave reduction is needed.  Each wave first issues the weight loads
// of its first two row pairs, then the workgroup builds the permuted activation layout
// once in LDS (every wave reads it back per segment), and the pair loop is software
// pipelined: the loads of pair p + 2*nw are issued as soon as pair p's registers are free.
// Launch shape of the row kernel (compile-time): waves per workgroup and the cap on
// workgroups per CU used to size the grid.
// Launch shape of the row kernel: 4-wave workgroups (one wave per SIMD), at most
// kRowWgPerCu per CU; waves loop over row pairs.  Measured on MI355X at K=N=6144 this
// beats both thinner grids (one pair per wave, staging repeated per 4 pairs) and fat
// 8/12-wave workgroups (one per CU, all waves held at the staging barriers).
constexpr int kRowWaves = 4;
constexpr int kRowWgPerCu = 2;

template <int NSEG>
struct RowBuf {
    Raw r[NSEG];
};

template <int NSEG>
__device__ __forceinline__ void rows_load(RowBuf<NSEG>& b, const uint8_t* row, const Geo& G, const int (&blkc)[NSEG]) {
#pragma unroll
    for (int s = 0; s < NSEG; ++s) b.r[s] = raw_load(row + (int64_t)blkc[s] * 144, G);
}

template <int NSEG>
__device__ __forceinline__ float rows_part(const RowBuf<NSEG>& b, const uint4* sxa, const float2* ssum,
                                           const Geo& G, const bool (&ok)[NSEG]) {
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
        Act A;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 q = sxa[(s * 8 + i) * 32 + G.s];
            A.xa[4 * i] = q.x;
            A.xa[4 * i + 1] = q.y;
            A.xa[4 * i + 2] = q.z;
            A.xa[4 * i + 3] = q.w;
        }
        const float2 sm = ssum[s * 32 + G.s];
        A.alo = sm.x;
        A.ahi = sm.y;
        const Hdr H = hdr_decode(b.r[s].h, G);
        float Slo, Shi;
        code_dots(b.r[s], A, Slo, Shi);
        const float v = lane_part(H, Slo, Shi, A);
        part += ok[s] ? v : 0.f;
        // keep the compiler from hoisting the next segment's LDS reads above this
        // segment's math: 161 instead of 222 VGPRs, i.e. 3 waves per SIMD
        __builtin_amdgcn_sched_barrier(0);
    }
    return part;
}

template <int NSEG, class Items, class Epi>
__global__ __launch_bounds__(kRowWaves * 64) void k_rows(Items items, Epi epi, const uint16_t* __restrict__ X,
                                                        int nsb, int64_t npairs) {
    __shared__ uint4 snat[NSEG * 256];          // activations in natural order (8 bf16 per entry)
    __shared__ uint4 sxa[NSEG * 8 * 32];        // activations in the lanes' dot2 order
    __shared__ float2 ssum[NSEG * 32];          // per-lane sub-block activation sums
    const int lane = threadIdx.x & 63;
    const Geo G = make_geo(lane);
    const int64_t nw = (int64_t)gridDim.x * kRowWaves;
    const int64_t p0 = (int64_t)blockIdx.x * kRowWaves + (threadIdx.x >> 6);
    int blkc[NSEG];
    bool ok[NSEG];
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
        const int blk = s * kSegBlocks + G.bs;
        ok[s] = blk < nsb;
        blkc[s] = ok[s] ? blk : 0;
    }
    // Row addresses first: for routed experts they depend on a load of the expert id.
    const int e_a = items.expert(p0), e_b = items.expert(p0 + nw);
    const uint8_t* row_a = items.row_e(p0, G.half, e_a);
    const uint8_t* row_b = items.row_e(p0 + nw, G.half, e_b);
    __builtin_amdgcn_sched_barrier(0);

    // Activations: every thread loads NSEG 16-B pieces of x, unconditionally (clamped
    // address, masked value), before any weight load.  Vector loads complete in order, so
    // storing them to LDS below waits only for these small cache-resident loads, never for
    // the weight stream, and no workgroup waits at the barriers for HBM.
    static_assert(kRowWaves == 4, "the activation staging assumes 256 threads");
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, (uint32_t)nsb * QK_K * 2u);   // 0 beyond K
    uint4 xv[NSEG];
#pragma unroll
    for (int j = 0; j < NSEG; ++j) xv[j] = buf_load16(xr, 16u * (threadIdx.x + 256u * j));
    __builtin_amdgcn_sched_barrier(0);

    // Unconditional (Items::row clamps out-of-range pairs to a valid row).
    RowBuf<NSEG> ba, bb;
    rows_load(ba, row_a, G, blkc);
    rows_load(bb, row_b, G, blkc);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int j = 0; j < NSEG; ++j) snat[threadIdx.x + 256 * j] = xv[j];
    __syncthreads();
    if (threadIdx.x < NSEG * 32) {
        const int st_s = threadIdx.x >> 5, st_l = threadIdx.x & 31;
        const Geo g2 = make_geo(st_l);
        const int base = ((st_s * kSegBlocks + g2.bs) * QK_K + 64 * g2.g) / 8;
        uint32_t xs[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint4 v = snat[base + i];
            xs[4 * i] = v.x;
            xs[4 * i + 1] = v.y;
            xs[4 * i + 2] = v.z;
            xs[4 * i + 3] = v.w;
        }
        Act A;
        act_from_natural(A, xs);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            sxa[(st_s * 8 + i) * 32 + st_l] =
                make_uint4(A.xa[4 * i], A.xa[4 * i + 1], A.xa[4 * i + 2], A.xa[4 * i + 3]);
        ssum[st_s * 32 + st_l] = make_float2(A.alo, A.ahi);
    }
    __syncthreads();

    for (int64_t p = p0; p < npairs; p += 2 * nw) {
        float tot = half_sum_dpp(rows_part<NSEG>(ba, sxa, ssum, G, ok));
        if (p + 2 * nw < npairs) rows_load(ba, items.row(p + 2 * nw, G.half), G, blkc);
        float other = __shfl(tot, 31, 64);
        if (lane == 63) epi(p, other, tot);
        const int64_t q = p + nw;
        if (q >= npairs) break;
        tot = half_sum_dpp(rows_part<NSEG>(bb, sxa, ssum, G, ok));
        if (q + 2 * nw < npairs) rows_load(bb, items.row(q + 2 * nw, G.half), G, blkc);
        other = __shfl(tot, 31, 64);
        if (lane == 63) epi(q, other, tot);
    }
}

// ------------------------------------------------------ MoE down (row tasks)
// A wave owns whole output rows d.  Row d needs one item per slot (expert e_s's row d
// against h[s]); a pass handles two slots (one per half-wave), so a row takes
// NP = ceil(nslots / 2) passes.  Passes are software pipelined two deep across the wave's
// whole (row, pass) sequence.  All slots' activations are permuted into the lane layout
// once per workgroup in LDS.  After each pass lane 63 folds the two slot results into the
// row's fp32 combine in slot order
//     facc = f32(facc + f32(g_s * bf16(y_s)))   (tools/glm_model_q4k_ref.py:799-809)
// (g = 1 for the shared-expert slot, i.e. facc + y_sh) and writes bf16(facc) after the
// row's last pass.  In passthrough mode (a single expert) y is bf16(y_0) itself.
struct DownRowsArgs {
    int nsb, nslots, topk, E, np, passthrough;
    int64_t H, I, ebytes, rb;
};

template <int NSEG>
struct DownBuf {
    Raw r[NSEG];
};

// Expert of pass q's slot for this lane's half-wave (loaded from the router's output).
__device__ __forceinline__ int down_expert(const int32_t* sel, const DownRowsArgs& a, int q, const Geo& G) {
    int s = 2 * q + G.half;
    s = s < a.nslots ? s : a.nslots - 1;
    // a buffer load (0 beyond the topk entries) rather than a branch around a load
    const int e = (int)buf_load4(buf_rsrc(sel, 4u * (uint32_t)a.topk), 4u * (uint32_t)s);
    return e < 0 ? 0 : (e >= a.E ? a.E - 1 : e);
}

__device__ __forceinline__ const uint8_t* down_row_e(const uint8_t* D, const uint8_t* shD, const DownRowsArgs& a,
                                                     int64_t d, int q, const Geo& G, int e) {
    int s = 2 * q + G.half;
    s = s < a.nslots ? s : a.nslots - 1;
    return (s < a.topk ? D + (int64_t)e * a.ebytes : shD) + d * a.rb;
}

__device__ __forceinline__ const uint8_t* down_row(const uint8_t* D, const uint8_t* shD, const int32_t* sel,
                                                   const DownRowsArgs& a, int64_t d, int q, const Geo& G) {
    return down_row_e(D, shD, a, d, q, G, down_expert(sel, a, q, G));
}

template <int NSEG>
__device__ __forceinline__ void down_load(DownBuf<NSEG>& b, const uint8_t* row, const Geo& G, const int (&blkc)[NSEG]) {
#pragma unroll
    for (int g = 0; g < NSEG; ++g) b.r[g] = raw_load(row + (int64_t)blkc[g] * 144, G);
}

template <int NSEG>
__global__ __launch_bounds__(256) void k_down_rows(const uint8_t* __restrict__ D, const uint8_t* __restrict__ shD,
                                                   const int32_t* __restrict__ sel,
                                                   const uint16_t* __restrict__ selw,
                                                   const uint16_t* __restrict__ hbuf, uint16_t* __restrict__ Y,
                                                   DownRowsArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int units = a.nslots * NSEG * 32;
    uint4* lxa = (uint4*)smem;                              // [slot*NSEG + seg][8][32]
    float2* lsum = (float2*)(smem + (size_t)units * 128);  // [slot*NSEG + seg][32]
    const int lane = threadIdx.x & 63;
    const Geo G = make_geo(lane);
    const int64_t nw = (int64_t)gridDim.x * (blockDim.x >> 6);
    const int64_t w0 = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    int blkc[NSEG];
    bool ok[NSEG];
#pragma unroll
    for (int g = 0; g < NSEG; ++g) {
        const int blk = g * kSegBlocks + G.bs;
        ok[g] = blk < a.nsb;
        blkc[g] = ok[g] ? blk : 0;
    }
    // this wave's units: rows d = w0 + k*nw, passes q = 0..np-1
    const int64_t nrows_w = w0 < a.H ? (a.H - w0 + nw - 1) / nw : 0;
    const int64_t nunits = nrows_w * a.np;

    // Row addresses of the first two units first: they depend on a load of the expert id.
    const int64_t dmax = a.H - 1;
    const int64_t d1r = w0 + (1 / a.np) * nw;
    const int e_a = down_expert(sel, a, 0, G), e_b = down_expert(sel, a, 1 % a.np, G);
    const uint8_t* row_a = down_row_e(D, shD, a, w0 < dmax ? w0 : dmax, 0, G, e_a);
    const uint8_t* row_b = down_row_e(D, shD, a, d1r < dmax ? d1r : dmax, 1 % a.np, G, e_b);

    // Activation staging: each thread owns at most two units (the launcher guarantees
    // units <= 2 * blockDim.x).  Their loads are issued before the weight loads so that
    // waiting for them does not wait for the weight stream (vector loads complete in order).
    uint32_t xs0[32], xs1[32];
    const int u0 = threadIdx.x, u1 = threadIdx.x + blockDim.x;
    auto unit_geo = [&](int u, int& sl, int& seg, int& ls) {
        sl = u / (NSEG * 32);
        const int rem = u - sl * NSEG * 32;
        seg = rem >> 5;
        ls = rem & 31;
    };
    {
        // buffer loads over h[nslots][I]: an invalid unit reads past the end and gets 0
        const __amdgpu_buffer_rsrc_t hr = buf_rsrc(hbuf, (uint32_t)(a.nslots * a.I * 2));
        auto unit_load = [&](int u, uint32_t (&xs)[32]) {
            int sl, seg, ls;
            unit_geo(u, sl, seg, ls);
            const Geo gg = make_geo(ls);
            const bool valid = u < units && seg * kSegBlocks + gg.bs < a.nsb;
            const uint32_t off = valid ? 2u * (uint32_t)(sl * a.I + (seg * kSegBlocks + gg.bs) * QK_K + 64 * gg.g)
                                       : 0x7FFFFFF0u;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 v = buf_load16(hr, off + 16u * i);
                xs[4 * i] = v.x;
                xs[4 * i + 1] = v.y;
                xs[4 * i + 2] = v.z;
                xs[4 * i + 3] = v.w;
            }
        };
        unit_load(u0, xs0);
        unit_load(u1, xs1);
    }
    __builtin_amdgcn_sched_barrier(0);   // keep the activation loads ahead of the weight loads

    // Unconditional loads (rows clamped into range) keep the activation wait static.
    DownBuf<NSEG> ba, bb;
    down_load(ba, row_a, G, blkc);
    down_load(bb, row_b, G, blkc);

    auto stage = [&](int u, const uint32_t (&xs)[32]) {
        int sl, seg, ls;
        unit_geo(u, sl, seg, ls);
        Act A;
        act_from_natural(A, xs);
        const int base = (u >> 5) * 256;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            lxa[base + i * 32 + ls] = make_uint4(A.xa[4 * i], A.xa[4 * i + 1], A.xa[4 * i + 2], A.xa[4 * i + 3]);
        lsum[u] = make_float2(A.alo, A.ahi);
    };
    if (u0 < units) stage(u0, xs0);
    if (u1 < units) stage(u1, xs1);
    __syncthreads();

    float facc = 0.f;
    auto step = [&](int64_t u, DownBuf<NSEG>& cur) {
        const int64_t r = u / a.np;
        const int q = (int)(u - r * a.np);
        const int64_t d = w0 + r * nw;
        int s = 2 * q + G.half;
        const bool svalid = s < a.nslots;
        s = svalid ? s : a.nslots - 1;
        float part = 0.f;
#pragma unroll
        for (int g = 0; g < NSEG; ++g) {
            const int ub = (s * NSEG + g) * 32;
            Act A;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 v = lxa[(ub >> 5) * 256 + i * 32 + G.s];
                A.xa[4 * i] = v.x;
                A.xa[4 * i + 1] = v.y;
                A.xa[4 * i + 2] = v.z;
                A.xa[4 * i + 3] = v.w;
            }
            const float2 sm = lsum[ub + G.s];
            A.alo = sm.x;
            A.ahi = sm.y;
            const Hdr Hh = hdr_decode(cur.r[g].h, G);
            float Slo, Shi;
            code_dots(cur.r[g], A, Slo, Shi);
            const float v = lane_part(Hh, Slo, Shi, A);
            part += ok[g] ? v : 0.f;
            __builtin_amdgcn_sched_barrier(0);
        }
        if (u + 2 < nunits) {
            const int64_t r2 = (u + 2) / a.np;
            down_load(cur, down_row(D, shD, sel, a, w0 + r2 * nw, (int)(u + 2 - r2 * a.np), G), G, blkc);
        }
        const float tot = half_sum_dpp(svalid ? part : 0.f);
        const float v0 = __shfl(tot, 31, 64);
        if (lane == 63) {
            const int s0 = 2 * q;
            if (a.passthrough) {
                Y[d] = (uint16_t)bf16_rne(v0);
            } else {
                const float y0 = bf16_to_f32(bf16_rne(v0));
                const float p0 = (s0 < a.topk ? bf16_to_f32(selw[s0]) : 1.0f) * y0;
                facc = facc + p0;
                if (s0 + 1 < a.nslots) {
                    const float y1 = bf16_to_f32(bf16_rne(tot));
                    const float p1 = (s0 + 1 < a.topk ? bf16_to_f32(selw[s0 + 1]) : 1.0f) * y1;
                    facc = facc + p1;
                }
                if (q == a.np - 1) {
                    Y[d] = (uint16_t)bf16_rne(facc);
                    facc = 0.f;
                }
            }
        }
    };
    for (int64_t u = 0; u < nunits; u += 2) {
        step(u, ba);
        if (u + 1 >= nunits) break;
        step(u + 1, bb);
    }
}

int g_cu_count = 0;

}  // namespace

int device_cu_count() {
    if (g_cu_count == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            g_cu_count = n;
        else
            g_cu_count = 256;
    }
    return g_cu_count;
}

namespace {

StreamGeom plan_stream(int64_t npairs, int64_t K, int passes) {
    StreamGeom sg;
    sg.nsb = (int)(K / QK_K);
    sg.nseg = (sg.nsb + kSegBlocks - 1) / kSegBlocks;
    sg.segw = sg.nseg < kMaxWaves ? sg.nseg : kMaxWaves;
    sg.spw = (sg.nseg + sg.segw - 1) / sg.segw;
    sg.rgc = sg.segw >= 4 ? 1 : (4 + sg.segw - 1) / sg.segw;
    sg.npairs = npairs;
    const int64_t target_wg = 2LL * device_cu_count();
    const int64_t per_batch = (int64_t)sg.rgc * passes;
    int64_t nb = (npairs + per_batch * target_wg - 1) / (per_batch * target_wg);
    sg.nbatch = (int)(nb < 1 ? 1 : nb);
    return sg;
}

inline unsigned wg_count(const StreamGeom& sg, int passes) {
    const int64_t per_wg = (int64_t)sg.rgc * passes * sg.nbatch;
    return (unsigned)((sg.npairs + per_wg - 1) / per_wg);
}

template <int TYPE, int MC, int PASSES, class Items, class Epi>
hipError_t run_stream(const Items& items, const Epi& epi, const uint16_t* X, int64_t K, int mrows, int64_t npairs,
                      hipStream_t st) {
    const StreamGeom sg = plan_stream(npairs, K, PASSES);
    const dim3 grid(wg_count(sg, PASSES));
    const dim3 block(64 * sg.segw * sg.rgc);
    hipLaunchKernelGGL((k_stream<TYPE, MC, PASSES, Items, Epi>), grid, block, 0, st, items, epi, X, K, mrows, sg);
    return hipGetLastError();
}

template <class Items, class Epi>
hipError_t run_rows(const Items& items, const Epi& epi, const uint16_t* X, int64_t K, int64_t npairs, hipStream_t st) {
    const int nsb = (int)(K / QK_K);
    const int nseg = (nsb + kSegBlocks - 1) / kSegBlocks;
    int64_t nwg = (npairs + kRowWaves - 1) / kRowWaves;
    const int64_t cap = (int64_t)kRowWgPerCu * device_cu_count();
    if (nwg > cap) nwg = cap;
    const dim3 grid((unsigned)nwg), block(kRowWaves * 64);
    switch (nseg) {
        case 1: hipLaunchKernelGGL((k_rows<1, Items, Epi>), grid, block, 0, st, items, epi, X, nsb, npairs); break;
        case 2: hipLaunchKernelGGL((k_rows<2, Items, Epi>), grid, block, 0, st, items, epi, X, nsb, npairs); break;
        case 3: hipLaunchKernelGGL((k_rows<3, Items, Epi>), grid, block, 0, st, items, epi, X, nsb, npairs); break;
        case 4: hipLaunchKernelGGL((k_rows<4, Items, Epi>), grid, block, 0, st, items, epi, X, nsb, npairs); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Epilogue of the row kernel for a plain GEMV (one activation row).
struct RowsPlainEpi {
    uint16_t* Y;
    float* Yf;
    int64_t N;
    __device__ void operator()(int64_t pair, float v0, float v1) const {
        const int64_t r = 2 * pair;
        Y[r] = (uint16_t)bf16_rne(v0);
        if (Yf) Yf[r] = v0;
        if (r + 1 < N) {
            Y[r + 1] = (uint16_t)bf16_rne(v1);
            if (Yf) Yf[r + 1] = v1;
        }
    }
};

struct RowsGateUpEpi {
    uint16_t* h;
    __device__ void operator()(int64_t pair, float v0, float v1) const {
        const uint32_t g = bf16_rne(v0), u = bf16_rne(v1);
        h[pair] = (uint16_t)bf16_rne(bf16_to_f32(glm_silu_bf16(g)) * bf16_to_f32(u));
    }
};

template <int TYPE, int PASSES>
hipError_t gemv_stream_mc(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                          float* yf, hipStream_t st) {
    const PlainItems items{W, N, row_bytes(TYPE, K)};
    const int64_t npairs = (N + 1) / 2;
    if (TYPE == T_Q4_K && M == 1 && K <= 4 * kSegWeights)
        return run_rows(items, RowsPlainEpi{y, yf, N}, x, K, npairs, st);
    hipError_t e = hipSuccess;
    for (int64_t m0 = 0; m0 < M && e == hipSuccess; m0 += 4) {
        const int mr = (int)((M - m0) < 4 ? (M - m0) : 4);
        const PlainEpi epi{y + m0 * N, yf ? yf + m0 * N : nullptr, N, mr};
        const uint16_t* xm = x + m0 * K;
        switch (mr) {
            case 1: e = run_stream<TYPE, 1, PASSES>(items, epi, xm, K, mr, npairs, st); break;
            case 2: e = run_stream<TYPE, 2, PASSES>(items, epi, xm, K, mr, npairs, st); break;
            case 3: e = run_stream<TYPE, 3, (PASSES > 1 ? PASSES / 2 : 1)>(items, epi, xm, K, mr, npairs, st); break;
            default: e = run_stream<TYPE, 4, (PASSES > 1 ? PASSES / 2 : 1)>(items, epi, xm, K, mr, npairs, st); break;
        }
    }
    return e;
}

}  // namespace

hipError_t launch_gemv_fast(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                            float* y_f32, hipStream_t st, bool dense) {
    switch (type) {
        case T_Q4_K:
            // the matrix-core dispatch serves every M wherever it serves one row (rows without a
            // multi-row kernel in the one-row order run one launch each)
            if (gemv_mfma_supported(N, K, 1)) return launch_gemv_mfma(w, N, K, x, M, y, y_f32, N, st, dense);
            return gemv_stream_mc<T_Q4_K, 4>((const uint8_t*)w, N, K, x, M, y, y_f32, st);
        case T_BF16: return gemv_stream_mc<T_BF16, 2>((const uint8_t*)w, N, K, x, M, y, y_f32, st);
        case T_Q6_K:
        case T_Q8_0:
        case T_F16: {
            // one tile covering all N rows; the activation rows share each weight pass
            if (!gemv_mixed_supported(type, K)) return hipErrorInvalidValue;
            const aipu_tile_desc d{type, 0, w, 0, N};
            return launch_gemv_mixed(&d, 1, K, x, M, y, y_f32, N, st);
        }
        default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------- MoE fast legs
hipError_t launch_moe_gateup_fast(const uint8_t* G, const uint8_t* U, const uint8_t* shG, const uint8_t* shU,
                                  const int32_t* sel, int topk, int nslots, int64_t E, int64_t H, int64_t I,
                                  const uint16_t* x, uint16_t* h, hipStream_t st) {
    const int64_t rb = row_bytes(T_Q4_K, H);
    const GateUpItems items{G, U, shG, shU, sel, topk, nslots, (int)I, (int)E, rb * I, rb};
    const int64_t npairs = (int64_t)nslots * I;
    if (H <= 4 * kSegWeights) return run_rows(items, RowsGateUpEpi{h}, x, H, npairs, st);
    const GateUpEpi epi{h, npairs};
    return run_stream<T_Q4_K, 1, 4>(items, epi, x, H, 1, npairs, st);
}

int64_t moe_down_lds_bytes(int nslots, int64_t I) {
    const int nseg = (int)((I / QK_K + kSegBlocks - 1) / kSegBlocks);
    return (int64_t)nslots * nseg * 32 * 136;
}

#ifndef AIPU_DOWN_WG_PER_CU
#define AIPU_DOWN_WG_PER_CU 2
#endif

hipError_t launch_moe_down_fast(const uint8_t* D, const uint8_t* shD, const int32_t* sel, const uint16_t* selw,
                                int topk, int nslots, int64_t E, int64_t H, int64_t I, const uint16_t* h, uint16_t* y,
                                int passthrough, hipStream_t st) {
    DownRowsArgs a;
    a.nsb = (int)(I / QK_K);
    const int nseg = (a.nsb + kSegBlocks - 1) / kSegBlocks;
    a.nslots = nslots;
    a.topk = topk;
    a.E = (int)E;
    a.np = (nslots + 1) / 2;
    a.passthrough = passthrough;
    a.H = H;
    a.I = I;
    a.rb = row_bytes(T_Q4_K, I);
    a.ebytes = a.rb * H;
    const int64_t lds = moe_down_lds_bytes(nslots, I);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const int waves = 4;
    if ((int64_t)nslots * nseg * 32 > 2 * 64 * waves) return hipErrorInvalidValue;   // <= 2 staging units per thread
    int64_t nwg = (H + waves - 1) / waves;
    const int64_t cap = (int64_t)AIPU_DOWN_WG_PER_CU * device_cu_count();
    if (nwg > cap) nwg = cap;
    const dim3 grid((unsigned)nwg), block(64 * waves);
    switch (nseg) {
        case 1: hipLaunchKernelGGL(k_down_rows<1>, grid, block, (size_t)lds, st, D, shD, sel, selw, h, y, a); break;
        case 2: hipLaunchKernelGGL(k_down_rows<2>, grid, block, (size_t)lds, st, D, shD, sel, selw, h, y, a); break;
        case 3: hipLaunchKernelGGL(k_down_rows<3>, grid, block, (size_t)lds, st, D, shD, sel, selw, h, y, a); break;
        case 4: hipLaunchKernelGGL(k_down_rows<4>, grid, block, (size_t)lds, st, D, shD, sel, selw, h, y, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace aipu
