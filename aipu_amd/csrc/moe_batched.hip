// MoE decode step for M activation rows (spec-verify / continuous batching).
//
// M = 1 is the single-row step of moe.hip (routed experts combined in slot order).  M > 1
// follows the PE_M > 1 union-skip path of src/glm_decoder_block_q4k.v:530-560,836-906: the
// expert axis is scanned in ascending index, only experts that some row selected are
// evaluated (their weights fetched once for all rows), and each row accumulates
// facc += f32(gate * bf16(y_e)) only for the experts it selected, in ascending expert index,
// then adds the shared expert with weight 1; fbuf = bf16(facc).
//
// Fast mode (Q4_K, up to 8 rows per pass, 2 where the union legs fit the small-batch
// kernel): router logits for all rows, one routing decision per row, a one-wave union pass,
// gate/up and down matrix-core GEMVs over the union slots (the grid is sized for the largest
// possible union; workgroups past the live slot count return at once), h = bf16(silu(g) * u)
// (fused into gate/up for two-row passes), and a per-row combine.  Reference mode runs each row
// through the single-row reference path with its routing reordered by expert index.
#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"
#include "route.hpp"

namespace aipu {
namespace {

constexpr int kRowsPerPass = 8;
constexpr int64_t kAlign = 256;
inline int64_t up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }
constexpr uint32_t kInactive = 0xFFFFFFFFu;   // no bf16-widened gate has this pattern

int max_union_slots(int64_t E, int topk, bool shared) {
    const int64_t u = (int64_t)kRowsPerPass * topk < E ? (int64_t)kRowsPerPass * topk : E;
    return (int)u + (shared ? 1 : 0);
}

struct BLayout {
    int64_t logits, sel, selw, uidx, nslots, ugate, gu, h, y, single, total;
};

BLayout b_layout(int64_t E, int64_t H, int64_t I, int topk) {
    const int ms = max_union_slots(E, topk, true);
    BLayout L;
    int64_t o = 0;
    L.logits = o; o += up(kRowsPerPass * E * 2);
    L.sel = o;    o += up(kRowsPerPass * topk * 4);
    L.selw = o;   o += up(kRowsPerPass * topk * 2);
    L.uidx = o;   o += up((int64_t)ms * 4);
    L.nslots = o; o += up(4);
    L.ugate = o;  o += up((int64_t)kRowsPerPass * ms * 4);
    L.gu = o;     o += up((int64_t)ms * 2 * kRowsPerPass * I * 2);
    L.h = o;      o += up((int64_t)ms * kRowsPerPass * I * 2);
    L.y = o;      o += up((int64_t)ms * kRowsPerPass * H * 2);
    L.single = o; o += moe_workspace_bytes(E, H, I, topk);   // reference path, one row at a time
    L.total = o;
    return L;
}

// Union of the M rows' experts in ascending index (one wave): uidx[0..nu), then -1 for the
// shared expert; *nslots = nu (+1); ugate[r][u] = the row's gate for union slot u (fp32
// bits of its bf16 sel_w) or kInactive.
__global__ __launch_bounds__(64) void k_union(const int32_t* __restrict__ sel, const uint16_t* __restrict__ selw,
                                              int M, int topk, int E, int shared, int ms, int32_t* __restrict__ uidx,
                                              int32_t* __restrict__ nslots, uint32_t* __restrict__ ugate) {
    __shared__ uint8_t flag[4096];
    __shared__ int32_t ulist[kRowsPerPass * 32];
    const int lane = threadIdx.x;
    for (int e = lane; e < E; e += 64) flag[e] = 0;
    __syncthreads();
    for (int i = lane; i < M * topk; i += 64) {
        const int e = sel[i];
        if (e >= 0 && e < E) flag[e] = 1;
    }
    __syncthreads();
    int count = 0;
    for (int c = 0; c < E; c += 64) {
        const int e = c + lane;
        const bool f = e < E && flag[e];
        const uint64_t b = __ballot(f);
        const int pos = count + __popcll(b & ((1ull << lane) - 1ull));
        if (f) {
            uidx[pos] = e;
            ulist[pos] = e;
        }
        count += __popcll(b);
    }
    __syncthreads();
    if (lane == 0) {
        if (shared) uidx[count] = -1;
        *nslots = count + (shared ? 1 : 0);
    }
    for (int i = lane; i < M * count; i += 64) {
        const int r = i / count, u = i - r * count;
        uint32_t g = kInactive;
        for (int t = 0; t < topk; ++t)
            if (sel[r * topk + t] == ulist[u]) g = (uint32_t)selw[r * topk + t] << 16;
        ugate[r * ms + u] = g;
    }
}

// The routing of every row of a pass and their union in one workgroup, for E <= kRouteMaxE:
// wave r routes row r (route.hpp's decision on keys it forms itself, the winners and slot
// weights one per lane); then the union of k_union over the decisions held in
// LDS.  One launch instead of two.
constexpr int kRUThreads = 64 * kRowsPerPass;
__global__ __launch_bounds__(kRUThreads) void k_route_union(const uint16_t* __restrict__ logits, int M, int E,
                                                            int topk, uint32_t scale_bits, int32_t* __restrict__ sel,
                                                            uint16_t* __restrict__ selw, int32_t* sel2, uint16_t* selw2,
                                                            int shared, int ms, int32_t* __restrict__ uidx,
                                                            int32_t* __restrict__ nslots, uint32_t* __restrict__ ugate) {
    __shared__ int32_t s_sel[kRowsPerPass * kRouteMaxTopk];
    __shared__ uint16_t s_selw[kRowsPerPass * kRouteMaxTopk];
    __shared__ uint8_t flag[kRouteMaxE];
    __shared__ int32_t ulist[kRowsPerPass * kRouteMaxTopk];
    __shared__ int s_count;
    const int t = threadIdx.x, nthr = blockDim.x, lane = t & 63;
    const int r = __builtin_amdgcn_readfirstlane(t >> 6);
    uint32_t lb[kRouteKeysPerLane];   // this wave's row of logits, loaded before the barrier
#pragma unroll
    for (int j = 0; j < kRouteKeysPerLane; ++j) {
        const int e = lane + 64 * j;
        lb[j] = r < M && e < E ? logits[(int64_t)r * E + e] : 0u;
    }
    for (int e = t; e < E; e += nthr) flag[e] = 0;
    __syncthreads();
    if (r < M) {
        uint32_t k[kRouteKeysPerLane];
#pragma unroll
        for (int j = 0; j < kRouteKeysPerLane; ++j) {
            const int e = lane + 64 * j;
            k[j] = e < E ? route_key(lb[j], e) : 0u;   // 0 is below every key
        }
        const uint32_t wl = route_tournament_lanes(k, topk, lane);
        int32_t sl;
        uint16_t swl;
        route_weights_wave(wl, topk, scale_bits, lane, sl, swl);
        if (lane < topk) {
            const int i = r * topk + lane;
            s_sel[i] = sl;
            s_selw[i] = swl;
            sel[i] = sl;
            selw[i] = swl;
            if (sel2) sel2[i] = sl;
            if (selw2) selw2[i] = swl;
            if (sl >= 0 && sl < E) flag[sl] = 1;
        }
    }
    __syncthreads();
    if (t < 64) {   // one wave lists the flagged experts in ascending index
        int count = 0;
        for (int c = 0; c < E; c += 64) {
            const int e = c + t;
            const bool f = e < E && flag[e];
            const uint64_t b = __ballot(f);
            const int pos = count + __popcll(b & ((1ull << t) - 1ull));
            if (f) {
                uidx[pos] = e;
                ulist[pos] = e;
            }
            count += __popcll(b);
        }
        if (t == 0) {
            if (shared) uidx[count] = -1;
            *nslots = count + (shared ? 1 : 0);
            s_count = count;
        }
    }
    __syncthreads();
    const int count = s_count;
    for (int i = t; i < M * count; i += nthr) {
        const int rr = i / count, u = i - rr * count;
        uint32_t g = kInactive;
        for (int q = 0; q < topk; ++q)
            if (s_sel[rr * topk + q] == ulist[u]) g = (uint32_t)s_selw[rr * topk + q] << 16;
        ugate[rr * ms + u] = g;
    }
}

// h[u][m][i] = bf16(f32(glm_silu(g)) * f32(up)) for the live slots.
__global__ void k_union_silu(const uint16_t* __restrict__ gu, const int32_t* __restrict__ nslots, int M, int64_t I,
                             int ms, uint16_t* __restrict__ h) {
    const int64_t per = (int64_t)M * I;
    const int64_t n = (int64_t)ms * per;
    const int live = *nslots;
    for (int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x) {
        const int u = (int)(j / per);
        if (u >= live) break;
        const int64_t k = j - (int64_t)u * per;
        const uint16_t g = gu[(int64_t)u * 2 * per + k];
        const uint16_t v = gu[(int64_t)u * 2 * per + per + k];
        h[j] = (uint16_t)bf16_rne(bf16_to_f32(glm_silu_bf16(g)) * bf16_to_f32(v));
    }
}

// out[m][d] = bf16(facc), facc over the routed union slots in ascending expert index (only
// the row's own experts), then the shared slot with weight 1; resid (nullable) added after.
constexpr int kCombineChunk = 16;   // a two-row pass of top-8 routing has at most 16 union slots
__global__ void k_union_combine(const uint16_t* __restrict__ y, const uint32_t* __restrict__ ugate,
                                const int32_t* __restrict__ nslots, int shared, int M, int64_t H, int ms,
                                const uint16_t* __restrict__ resid, int64_t rstride, uint16_t* __restrict__ out,
                                int64_t ostride) {
    const int live = *nslots;
    const int nu = live - (shared ? 1 : 0);
    for (int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; j < (int64_t)M * H;
         j += (int64_t)gridDim.x * blockDim.x) {
        const int m = (int)(j / H);
        const int64_t d = j - (int64_t)m * H;
        float facc = 0.0f;
        // the gates and outputs of up to kCombineChunk slots are loaded before their adds, so one
        // memory round trip serves them (slots past the union reread the last one, unused)
        for (int u0 = 0; u0 < nu; u0 += kCombineChunk) {
            uint32_t g[kCombineChunk], yv[kCombineChunk];
#pragma unroll
            for (int k = 0; k < kCombineChunk; ++k) {
                const int u = u0 + k < nu ? u0 + k : nu - 1;
                g[k] = ugate[m * ms + u];
                yv[k] = y[((int64_t)u * M + m) * H + d];
            }
#pragma unroll
            for (int k = 0; k < kCombineChunk; ++k) {
                if (u0 + k >= nu || g[k] == kInactive) continue;
                const float p = __uint_as_float(g[k]) * bf16_to_f32(yv[k]);
                facc = facc + p;
            }
        }
        if (shared) facc = facc + bf16_to_f32(y[((int64_t)nu * M + m) * H + d]);
        uint32_t o = bf16_rne(facc);
        if (resid) o = bf16_rne(bf16_to_f32(resid[m * rstride + d]) + bf16_to_f32(o));
        out[m * ostride + d] = (uint16_t)o;
    }
}

hipError_t after_gateup(const MoeUnionArgs& a, hipStream_t st) {
    const int64_t n = (int64_t)a.max_slots * a.M * a.I;
    int64_t b = (n + 255) / 256;
    b = b < 1 ? 1 : (b > 2048 ? 2048 : b);
    hipLaunchKernelGGL(k_union_silu, dim3((unsigned)b), dim3(256), 0, st, a.gu, a.nslots, a.M, a.I, a.max_slots,
                       a.h);
    return hipGetLastError();
}

#define AIPU_TRY(x)                         \
    do {                                    \
        hipError_t e_ = (x);                \
        if (e_ != hipSuccess) return e_;    \
    } while (0)

// One fast pass over M <= 8 rows starting at row r0.
hipError_t fast_pass(const MoeArgs& a, int64_t r0, int M, const BLayout& L, hipStream_t st) {
    uint8_t* ws = (uint8_t*)a.ws;
    uint16_t* logits = (uint16_t*)(ws + L.logits);
    int32_t* sel = (int32_t*)(ws + L.sel);
    uint16_t* selw = (uint16_t*)(ws + L.selw);
    int32_t* uidx = (int32_t*)(ws + L.uidx);
    int32_t* nsl = (int32_t*)(ws + L.nslots);
    uint32_t* ugate = (uint32_t*)(ws + L.ugate);
    const uint16_t* x = a.x + r0 * a.H;
    const bool shared = a.sh_gate != nullptr;
    const int ms = max_union_slots(a.E, a.topk, shared);

    // router logits [M][E]
    if (a.router_type == T_BF16) {
        AIPU_TRY(launch_router_bf16_logits_rows((const uint16_t*)a.router_w, x, a.H, (int)a.E, M, logits, st));
    } else if (a.router_type == T_Q4_K && gemv_mfma_supported(a.E, a.H, M)) {
        AIPU_TRY(launch_gemv_mfma(a.router_w, a.E, a.H, x, M, logits, nullptr, a.E, st));
    } else if (a.router_type == T_Q4_K || gemv_mixed_supported(a.router_type, a.H)) {
        AIPU_TRY(launch_gemv_fast(a.router_type, a.router_w, a.E, a.H, x, M, logits, nullptr, st));
    } else {   // past the mixed-type kernel's staging limit: the exact kernel (within any tolerance)
        AIPU_TRY(launch_gemv_ref(a.router_type, a.router_w, a.E, a.H, x, M, logits, nullptr, st));
    }
    int32_t* sel2 = a.sel_idx_out ? a.sel_idx_out + r0 * a.topk : nullptr;
    uint16_t* selw2 = a.sel_w_out ? a.sel_w_out + r0 * a.topk : nullptr;
    if (a.E <= kRouteMaxE && a.topk <= kRouteMaxTopk) {
        hipLaunchKernelGGL(k_route_union, dim3(1), dim3(kRUThreads), 0, st, logits, M, (int)a.E, a.topk, a.scale_bits,
                           sel, selw, sel2, selw2, shared ? 1 : 0, ms, uidx, nsl, ugate);
    } else {
        AIPU_TRY(launch_router_tail_rows(logits, M, (int)a.E, a.topk, a.scale_bits, sel, selw, sel2, selw2, st));
        hipLaunchKernelGGL(k_union, dim3(1), dim3(64), 0, st, sel, selw, M, a.topk, (int)a.E, shared ? 1 : 0, ms, uidx,
                           nsl, ugate);
    }
    AIPU_TRY(hipGetLastError());
    MoeUnionArgs u;
    u.G = a.gate_exps;
    u.U = a.up_exps;
    u.D = a.down_exps;
    u.shG = a.sh_gate;
    u.shU = a.sh_up;
    u.shD = a.sh_down;
    u.uidx = uidx;
    u.nslots = nsl;
    u.max_slots = ms;
    u.M = M;
    u.H = a.H;
    u.I = a.I;
    u.x = x;
    u.gu = (uint16_t*)(ws + L.gu);
    u.h = (uint16_t*)(ws + L.h);
    u.y = (uint16_t*)(ws + L.y);
    u.after_gateup_fn = after_gateup;
    AIPU_TRY(launch_moe_union_mfma(u, st));
    int64_t b = ((int64_t)M * a.H + 255) / 256;
    b = b > 1024 ? 1024 : b;
    hipLaunchKernelGGL(k_union_combine, dim3((unsigned)b), dim3(256), 0, st, u.y, ugate, nsl, shared ? 1 : 0, M, a.H,
                       ms, a.resid ? a.resid + r0 * a.H : nullptr, a.H, a.y + r0 * a.H, a.H);
    return hipGetLastError();
}

}  // namespace

int64_t moe_batched_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk) {
    return b_layout(E, H, I, topk).total;
}

hipError_t launch_moe_decode_batched(const MoeArgs& a, int64_t M, hipStream_t st) {
    const BLayout L = b_layout(a.E, a.H, a.I, a.topk);
    uint8_t* ws = (uint8_t*)a.ws;
    const bool fast = a.mode == AIPU_MODE_FAST && a.type == T_Q4_K && a.E <= 4096 && a.topk <= 32;
    if (M == 1) {   // the single-row step (slot-order combine, PE_M == 1)
        MoeArgs m = a;
        m.ws = ws + L.single;
        return launch_moe_decode(m, st);
    }
    // passes of two rows where the union legs run on the small-batch kernel (fused SwiGLU):
    // per row, two-row unions cost less than wider ones on the slower kernels
    const int per = moe_union_pass_rows(a.H, a.I);
    int64_t r0 = 0;
    while (r0 < M) {
        const int rows = (int)(M - r0 < per ? M - r0 : per);
        // a leftover single row of the batch takes a one-row union pass too: the same kernels
        // and summation order as the batch's other rows (the single-row step's legs differ)
        if (fast && moe_union_supported(a.H, a.I, rows)) {
            AIPU_TRY(fast_pass(a, r0, rows, L, st));
        } else {
            // one row at a time with its experts reordered by index (still the M > 1 order)
            for (int r = 0; r < rows; ++r) {
                MoeArgs m = a;
                m.ws = ws + L.single;
                m.x = a.x + (r0 + r) * a.H;
                m.y = a.y + (r0 + r) * a.H;
                m.resid = a.resid ? a.resid + (r0 + r) * a.H : nullptr;
                m.sel_idx_out = a.sel_idx_out ? a.sel_idx_out + (r0 + r) * a.topk : nullptr;
                m.sel_w_out = a.sel_w_out ? a.sel_w_out + (r0 + r) * a.topk : nullptr;
                m.ascending = true;
                AIPU_TRY(launch_moe_decode(m, st));
            }
        }
        r0 += rows;
    }
    return hipSuccess;
}

}  // namespace aipu
