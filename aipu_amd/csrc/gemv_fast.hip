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
    __device__ const uint8_t* row(int64_t pair, int half) const {
        int64_t r = 2 * pair + half;
        r = r < N ? r : N - 1;
        return W + r * rb;
    }
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
    __device__ const uint8_t* row(int64_t pair, int half) const {
        const int npairs = nslots * I;
        int p = (int)(pair < npairs ? pair : npairs - 1);
        const int s = p / I;
        const int i = p - s * I;
        const uint8_t* base;
        if (s < topk) {
            int e = sel[s];
            e = e < 0 ? 0 : (e >= E ? E - 1 : e);
            base = (half ? U : G) + (int64_t)e * ebytes;
        } else {
            base = half ? shU : shG;
        }
        return base + (int64_t)i * rb;
    }
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

// ------------------------------------------------------------- MoE down
// Items are (output row d, slot s) flattened as d * nslots + s within the workgroup's
// rows.  Each slot's activations h[s] are permuted into the lane layout once per
// workgroup and kept in LDS; each item's bf16 result goes to LDS, and after the last
// batch every output row is combined in slot order:
//   facc = f32(facc + f32(g_s * y_s)),  y = bf16(facc)   (tools/glm_model_q4k_ref.py:799-809)
// with g = 1 for the shared-expert slot (adding y_sh directly, as the reference does).
constexpr int kDownPasses = 4;

struct DownGeom {
    int nsb, nseg, segw, rgc, nbatch;
    int rows_per_wg;
    int nslots, topk, E;
    int passthrough;   // single expert: y is the slot's bf16 output itself (no combine)
    int64_t H, I, ebytes, rb;
};

__global__ __launch_bounds__(kMaxWaves * 64) void k_moe_down(const uint8_t* __restrict__ D,
                                                             const uint8_t* __restrict__ shD,
                                                             const int32_t* __restrict__ sel,
                                                             const uint16_t* __restrict__ selw,
                                                             const uint16_t* __restrict__ hbuf,
                                                             uint16_t* __restrict__ Y, DownGeom dg) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red[2][kMaxWaves][kDownPasses][2];
    const int units = dg.nslots * dg.nseg * 32;
    uint4* lxa = (uint4*)smem;                                          // [unit/32][8][32] uint4
    float2* lsum = (float2*)(smem + (size_t)units * 128);              // [unit]
    float* ys = (float*)(smem + (size_t)units * 136);                  // [rows_per_wg][nslots]

    // 1. activations -> LDS in the lane layout
    for (int u = threadIdx.x; u < units; u += blockDim.x) {
        const int s = u / (dg.nseg * 32);
        const int rem = u - s * dg.nseg * 32;
        const int seg = rem >> 5, ls = rem & 31;
        Geo G = make_geo(ls);
        Act A;
        act_load(A, hbuf + (int64_t)s * dg.I, seg, G, seg * kSegBlocks + G.bs < dg.nsb);
        const int base = (u >> 5) * 256;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            lxa[base + i * 32 + ls] = make_uint4(A.xa[4 * i], A.xa[4 * i + 1], A.xa[4 * i + 2], A.xa[4 * i + 3]);
        lsum[u] = make_float2(A.alo, A.ahi);
    }
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rg = wave / dg.segw, wseg = wave - rg * dg.segw;
    const Geo G = make_geo(lane);
    const int64_t d0 = (int64_t)blockIdx.x * dg.rows_per_wg;
    const int nrows = (int)((dg.H - d0) < dg.rows_per_wg ? (dg.H - d0) : dg.rows_per_wg);
    const int nitems = nrows * dg.nslots;
    constexpr int VP = Pow2<kDownPasses>::v;
    constexpr int LV = Pow2<kDownPasses>::lg;

    int buf = 0;
    for (int b = 0; b < dg.nbatch; ++b) {
        const int it0 = ((rg * dg.nbatch) + b) * 2 * kDownPasses;
        float part[kDownPasses];
        int itm[kDownPasses];
#pragma unroll
        for (int p = 0; p < kDownPasses; ++p) {
            part[p] = 0.f;
            int it = it0 + 2 * p + G.half;
            itm[p] = it < nitems ? it : nitems - 1;
        }
        const int seg = wseg;
        const int blk = seg * kSegBlocks + G.bs;
        const bool bvalid = blk < dg.nsb;
        Raw r[kDownPasses];
#pragma unroll
        for (int p = 0; p < kDownPasses; ++p) {
            const int d = itm[p] / dg.nslots, s = itm[p] - (itm[p] / dg.nslots) * dg.nslots;
            const uint8_t* base;
            if (s < dg.topk) {
                int e = sel[s];
                e = e < 0 ? 0 : (e >= dg.E ? dg.E - 1 : e);
                base = D + (int64_t)e * dg.ebytes;
            } else {
                base = shD;
            }
            r[p] = raw_load(base + (d0 + d) * dg.rb + (int64_t)(bvalid ? blk : 0) * 144, G);
        }
#pragma unroll
        for (int p = 0; p < kDownPasses; ++p) {
            const int s = itm[p] % dg.nslots;
            const int u = (s * dg.nseg + seg) * 32 + G.s;
            Act A;
            const int base = (u >> 5) * 256;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint4 q = lxa[base + i * 32 + G.s];
                A.xa[4 * i] = q.x;
                A.xa[4 * i + 1] = q.y;
                A.xa[4 * i + 2] = q.z;
                A.xa[4 * i + 3] = q.w;
            }
            const float2 sm = lsum[u];
            A.alo = sm.x;
            A.ahi = sm.y;
            const Hdr H = hdr_decode(r[p].h, G);
            float Slo, Shi;
            code_dots(r[p], A, Slo, Shi);
            part[p] = bvalid ? lane_part(H, Slo, Shi, A) : 0.f;
        }
        float v[VP];
#pragma unroll
        for (int i = 0; i < VP; ++i) v[i] = i < kDownPasses ? part[i] : 0.f;
        const float tot = half_reduce<VP>(v, lane);
        const int vi = (G.s >> (5 - LV)) & (VP - 1);
        if ((G.s & ((32 >> LV) - 1)) == 0 && vi < kDownPasses) red[buf][wave][vi][G.half] = tot;
        __syncthreads();
        const int t = threadIdx.x;
        if (t < dg.rgc * kDownPasses * 2) {
            const int erg = t / (2 * kDownPasses), ev = t - erg * 2 * kDownPasses;
            const int p = ev >> 1, hf = ev & 1;
            float acc = 0.f;
            for (int w = 0; w < dg.segw; ++w) acc += red[buf][erg * dg.segw + w][p][hf];
            const int it = ((erg * dg.nbatch) + b) * 2 * kDownPasses + 2 * p + hf;
            if (it < nitems) ys[it] = bf16_to_f32(bf16_rne(acc));
        }
        buf ^= 1;
    }
    __syncthreads();
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        if (dg.passthrough) {
            Y[d0 + r] = (uint16_t)(__float_as_uint(ys[r * dg.nslots]) >> 16);
            continue;
        }
        float facc = 0.f;
        for (int s = 0; s < dg.nslots; ++s) {
            const float g = s < dg.topk ? bf16_to_f32(selw[s]) : 1.0f;
            const float prod = g * ys[r * dg.nslots + s];
            facc = facc + prod;
        }
        Y[d0 + r] = (uint16_t)bf16_rne(facc);
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

template <int TYPE, int PASSES>
hipError_t gemv_stream_mc(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                          float* yf, hipStream_t st) {
    const PlainItems items{W, N, row_bytes(TYPE, K)};
    const int64_t npairs = (N + 1) / 2;
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
                            float* y_f32, hipStream_t st) {
    switch (type) {
        case T_Q4_K: return gemv_stream_mc<T_Q4_K, 4>((const uint8_t*)w, N, K, x, M, y, y_f32, st);
        case T_BF16: return gemv_stream_mc<T_BF16, 2>((const uint8_t*)w, N, K, x, M, y, y_f32, st);
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
    const GateUpEpi epi{h, npairs};
    return run_stream<T_Q4_K, 1, 4>(items, epi, x, H, 1, npairs, st);
}

int64_t moe_down_lds_bytes(int nslots, int64_t I, int rows_per_wg) {
    const int nseg = (int)((I / QK_K + kSegBlocks - 1) / kSegBlocks);
    return (int64_t)nslots * nseg * 32 * 136 + (int64_t)rows_per_wg * nslots * 4;
}

hipError_t launch_moe_down_fast(const uint8_t* D, const uint8_t* shD, const int32_t* sel, const uint16_t* selw,
                                int topk, int nslots, int64_t E, int64_t H, int64_t I, const uint16_t* h, uint16_t* y,
                                int passthrough, hipStream_t st) {
    DownGeom dg;
    dg.passthrough = passthrough;
    dg.nsb = (int)(I / QK_K);
    dg.nseg = (dg.nsb + kSegBlocks - 1) / kSegBlocks;
    if (dg.nseg > kMaxWaves) return hipErrorInvalidValue;
    dg.segw = dg.nseg;
    dg.rgc = dg.segw >= 4 ? 1 : (4 + dg.segw - 1) / dg.segw;
    const int cus = device_cu_count();
    int rows = (int)((H + cus - 1) / cus);
    if (rows < 1) rows = 1;
    if (rows > 64) rows = 64;
    dg.rows_per_wg = rows;
    dg.nslots = nslots;
    dg.topk = topk;
    dg.E = (int)E;
    dg.H = H;
    dg.I = I;
    dg.rb = row_bytes(T_Q4_K, I);
    dg.ebytes = dg.rb * H;
    const int items = rows * nslots;
    const int per_batch = dg.rgc * 2 * kDownPasses;
    dg.nbatch = (items + per_batch - 1) / per_batch;
    const int64_t lds = moe_down_lds_bytes(nslots, I, rows);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((H + rows - 1) / rows));
    const dim3 block(64 * dg.segw * dg.rgc);
    hipLaunchKernelGGL(k_moe_down, grid, block, (size_t)lds, st, D, shD, sel, selw, h, y, dg);
    return hipGetLastError();
}

}  // namespace aipu
