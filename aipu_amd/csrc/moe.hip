// MoE SwiGLU decode step (M = 1): router GEMV -> router tail -> per-slot SwiGLU experts
// -> slot-ordered combine.  Mirrors the MoE half of decoder_block
// (tools/glm_model_q4k_ref.py:797-809) with moe_router (:663-681) and swiglu_expert
// (:702-708); RTL src/glm_decoder_block_q4k.v:494-497,636-650.
//
// AIPU_MODE_REF runs every GEMV in reference order (bit-exact to the oracle, any ggml
// type).  AIPU_MODE_FAST runs the streaming kernels: a bf16/Q4_K router GEMV, one fused
// gate/up kernel that also forms h = bf16(silu(gate) * up), and one down kernel that
// keeps all slots' h in LDS and combines the slots in order.  Everything is stream-ordered
// with no host synchronisation, so the whole step can be captured in a HIP graph.
#include "common.hpp"
#include "glm_act.hpp"
#include "launch.hpp"

namespace aipu {

hipError_t launch_moe_gateup_fast(const uint8_t* G, const uint8_t* U, const uint8_t* shG, const uint8_t* shU,
                                  const int32_t* sel, int topk, int nslots, int64_t E, int64_t H, int64_t I,
                                  const uint16_t* x, uint16_t* h, hipStream_t st);
hipError_t launch_moe_down_fast(const uint8_t* D, const uint8_t* shD, const int32_t* sel, const uint16_t* selw,
                                int topk, int nslots, int64_t E, int64_t H, int64_t I, const uint16_t* h, uint16_t* y,
                                int passthrough, hipStream_t st);
int64_t moe_down_lds_bytes(int nslots, int64_t I);

namespace {

constexpr int64_t kAlign = 256;
inline int64_t up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct WsLayout {
    int64_t logits, sel, selw, h, g, u, ys, facc, total;
};

WsLayout ws_layout(int64_t E, int64_t H, int64_t I, int topk) {
    const int64_t nslots = topk + 1;
    WsLayout L;
    int64_t o = 0;
    L.logits = o; o += up(E * 2);
    L.sel = o;    o += up(64 * 4);
    L.selw = o;   o += up(64 * 2);
    L.h = o;      o += up(nslots * I * 2);
    L.g = o;      o += up(nslots * I * 2);
    L.u = o;      o += up(nslots * I * 2);
    L.ys = o;     o += up(nslots * H * 2);
    L.facc = o;   o += up(H * 4);
    L.total = o;
    return L;
}

// h = bf16(f32(glm_silu(gate)) * f32(up)) elementwise (reference path).
__global__ void k_silu_mul(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u, int64_t n,
                           uint16_t* __restrict__ h) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        h[i] = (uint16_t)bf16_rne(bf16_to_f32(glm_silu_bf16(g[i])) * bf16_to_f32(u[i]));
}

// Slot-ordered combine (reference path): facc = f32(facc + f32(g_s * y_s)); shared slot
// (index topk, if present) adds y_s with weight 1.
__global__ void k_combine(const uint16_t* __restrict__ ys, const uint16_t* __restrict__ selw, int topk, int nslots,
                          int64_t H, uint16_t* __restrict__ y) {
    for (int64_t d = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; d < H; d += (int64_t)gridDim.x * blockDim.x) {
        float facc = 0.0f;
        for (int s = 0; s < nslots; ++s) {
            const float ye = bf16_to_f32(ys[(int64_t)s * H + d]);
            if (s < topk) {
                const float prod = bf16_to_f32(selw[s]) * ye;
                facc = facc + prod;
            } else {
                facc = facc + ye;
            }
        }
        y[d] = (uint16_t)bf16_rne(facc);
    }
}

// Reorder the routing decision (sel, selw) by ascending expert index (one thread; topk <= 32).
__global__ void k_sort_slots(int32_t* sel, uint16_t* selw, int topk) {
    if (threadIdx.x != 0) return;
    for (int i = 1; i < topk; ++i) {
        const int32_t e = sel[i];
        const uint16_t w = selw[i];
        int j = i - 1;
        for (; j >= 0 && sel[j] > e; --j) {
            sel[j + 1] = sel[j];
            selw[j + 1] = selw[j];
        }
        sel[j + 1] = e;
        selw[j + 1] = w;
    }
}

inline int blocks_for(int64_t n) {
    int64_t b = (n + 255) / 256;
    return (int)(b < 1 ? 1 : (b > 4096 ? 4096 : b));
}

}  // namespace

int64_t moe_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk) { return ws_layout(E, H, I, topk).total; }

#define AIPU_TRY(x)                         \
    do {                                    \
        hipError_t e_ = (x);                \
        if (e_ != hipSuccess) return e_;    \
    } while (0)

hipError_t launch_moe_decode(const MoeArgs& a, hipStream_t st) {
    const WsLayout L = ws_layout(a.E, a.H, a.I, a.topk);
    uint8_t* ws = (uint8_t*)a.ws;
    uint16_t* logits = (uint16_t*)(ws + L.logits);
    int32_t* sel = (int32_t*)(ws + L.sel);
    uint16_t* selw = (uint16_t*)(ws + L.selw);
    uint16_t* h = (uint16_t*)(ws + L.h);
    float* facc = (float*)(ws + L.facc);
    const bool has_shared = a.sh_gate != nullptr;
    const int nslots = a.topk + (has_shared ? 1 : 0);
    const bool fast = a.mode == AIPU_MODE_FAST && a.type == T_Q4_K;

    // 1. router logits
    if (a.logits_ready && a.mode == AIPU_MODE_FAST)
        ;   // formed by the caller's launch (the FFN half's router with its RMSNorm)
    else if (a.mode == AIPU_MODE_FAST && a.router_type == T_BF16)
        AIPU_TRY(launch_router_bf16_logits((const uint16_t*)a.router_w, a.x, a.H, (int)a.E, logits, st));
    else if (a.mode == AIPU_MODE_FAST && a.router_type == T_Q4_K)
        AIPU_TRY(launch_gemv_fast(a.router_type, a.router_w, a.E, a.H, a.x, 1, logits, nullptr, st));
    else
        AIPU_TRY(launch_gemv_ref(a.router_type, a.router_w, a.E, a.H, a.x, 1, logits, nullptr, st));

    // 2-3. fast path: the gate/up kernel routes from the logits in every workgroup and
    // publishes the decision for the down kernel (no separate router-tail launch)
    if (fast && !a.ascending && moe_persist_supported(a.E, a.topk, nslots, a.H, a.I)) {
        // persistent legs: one workgroup per CU streams every expert row once (shared expert last)
        const MoeRoute route{nullptr, logits, a.scale_bits, sel, selw, a.sel_idx_out, a.sel_w_out};
        AIPU_TRY(launch_moe_gateup_persist(a.gate_exps, a.up_exps, a.sh_gate, a.sh_up, a.down_exps, a.sh_down, route,
                                           a.topk, nslots, a.E, a.H, a.I, a.x, h, st));
        return launch_moe_down_persist(a.down_exps, a.sh_down, sel, selw, a.topk, nslots, a.E, a.H, a.I, h, a.y,
                                       a.resid, st);
    }
    if (fast && !a.ascending && moe_mfma_supported(nslots, a.H, a.I) && moe_route_in_kernel(a.E, a.topk, a.H)) {
        const MoeRoute route{nullptr, logits, a.scale_bits, sel, selw, a.sel_idx_out, a.sel_w_out};
        AIPU_TRY(launch_moe_gateup_mfma(a.gate_exps, a.up_exps, a.sh_gate, a.sh_up, route, a.topk, nslots, a.E, a.H,
                                        a.I, a.x, h, st));
        return launch_moe_down_mfma(a.down_exps, a.sh_down, sel, selw, a.topk, nslots, a.E, a.H, a.I, h, a.y, 0, st,
                                    facc, a.resid);
    }
    // 2. router tail (one wave), then the experts
    AIPU_TRY(launch_router_tail(logits, (int)a.E, a.topk, a.scale_bits, sel, selw, nullptr, st, a.sel_idx_out,
                                a.sel_w_out));
    if (a.ascending) {   // batched-row semantics: experts combined in ascending index order
        hipLaunchKernelGGL(k_sort_slots, dim3(1), dim3(64), 0, st, sel, selw, a.topk);
        AIPU_TRY(hipGetLastError());
    }
    if (fast && moe_mfma_supported(nslots, a.H, a.I)) {
        const MoeRoute route{sel, nullptr, 0u, nullptr, nullptr, nullptr, nullptr};
        AIPU_TRY(launch_moe_gateup_mfma(a.gate_exps, a.up_exps, a.sh_gate, a.sh_up, route, a.topk, nslots, a.E, a.H,
                                        a.I, a.x, h, st));
        return launch_moe_down_mfma(a.down_exps, a.sh_down, sel, selw, a.topk, nslots, a.E, a.H, a.I, h, a.y, 0, st,
                                    facc, a.resid);
    }
    if (fast) {
        AIPU_TRY(launch_moe_gateup_fast(a.gate_exps, a.up_exps, a.sh_gate, a.sh_up, sel, a.topk, nslots, a.E, a.H,
                                        a.I, a.x, h, st));
        AIPU_TRY(launch_moe_down_fast(a.down_exps, a.sh_down, sel, selw, a.topk, nslots, a.E, a.H, a.I, h, a.y, 0,
                                      st));
        return a.resid ? launch_residual_add(a.resid, a.y, a.H, a.y, st) : hipSuccess;
    }
    uint16_t* g = (uint16_t*)(ws + L.g);
    uint16_t* u = (uint16_t*)(ws + L.u);
    uint16_t* ys = (uint16_t*)(ws + L.ys);
    const int64_t rbH = row_bytes(a.type, a.H), rbI = row_bytes(a.type, a.I);
    AIPU_TRY(launch_gemv_ref_gather(a.type, a.gate_exps, a.I, a.H, a.x, 1, g, nullptr, nslots, sel, a.topk, a.E,
                                    rbH * a.I, a.sh_gate, 0, a.I, st));
    AIPU_TRY(launch_gemv_ref_gather(a.type, a.up_exps, a.I, a.H, a.x, 1, u, nullptr, nslots, sel, a.topk, a.E,
                                    rbH * a.I, a.sh_up, 0, a.I, st));
    hipLaunchKernelGGL(k_silu_mul, dim3(blocks_for(nslots * a.I)), dim3(256), 0, st, g, u, nslots * a.I, h);
    AIPU_TRY(hipGetLastError());
    AIPU_TRY(launch_gemv_ref_gather(a.type, a.down_exps, a.H, a.I, h, 1, ys, nullptr, nslots, sel, a.topk, a.E,
                                    rbI * a.H, a.sh_down, a.I, a.H, st));
    hipLaunchKernelGGL(k_combine, dim3(blocks_for(a.H)), dim3(256), 0, st, ys, selw, a.topk, nslots, a.H, a.y);
    AIPU_TRY(hipGetLastError());
    return a.resid ? launch_residual_add(a.resid, a.y, a.H, a.y, st) : hipSuccess;
}

// A single SwiGLU expert: the expert is treated as the (only) shared slot, so no router
// runs; y is the down GEMV output itself (no combine), as swiglu_expert returns it.
hipError_t launch_swiglu_expert(int type, const void* wg, const void* wu, const void* wd, int64_t H, int64_t I,
                                const uint16_t* x, uint16_t* y, uint16_t* h_out, int mode, void* wsp,
                                hipStream_t st) {
    const WsLayout L = ws_layout(1, H, I, 1);
    uint8_t* ws = (uint8_t*)wsp;
    uint16_t* h = h_out ? h_out : (uint16_t*)(ws + L.h);
    const uint8_t* G = (const uint8_t*)wg;
    const uint8_t* U = (const uint8_t*)wu;
    const uint8_t* D = (const uint8_t*)wd;
    if (mode == AIPU_MODE_FAST && type == T_Q4_K) {
        // No routing: the expert runs as the shared slot.  The kernels still read one
        // (ignored) expert id, so they get the workspace's id slot rather than a null pointer.
        const int32_t* no_sel = (const int32_t*)(ws + L.sel);
        if (moe_mfma_supported(1, H, I)) {
            const MoeRoute route{no_sel, nullptr, 0u, nullptr, nullptr, nullptr, nullptr};
            AIPU_TRY(launch_moe_gateup_mfma(G, U, G, U, route, 0, 1, 1, H, I, x, h, st));
            return launch_moe_down_mfma(D, D, no_sel, nullptr, 0, 1, 1, H, I, h, y, 1, st);
        }
        AIPU_TRY(launch_moe_gateup_fast(G, U, G, U, no_sel, 0, 1, 1, H, I, x, h, st));
        return launch_moe_down_fast(D, D, no_sel, nullptr, 0, 1, 1, H, I, h, y, 1, st);
    }
    uint16_t* g = (uint16_t*)(ws + L.g);
    uint16_t* u = (uint16_t*)(ws + L.u);
    AIPU_TRY(launch_gemv_ref(type, wg, I, H, x, 1, g, nullptr, st));
    AIPU_TRY(launch_gemv_ref(type, wu, I, H, x, 1, u, nullptr, st));
    hipLaunchKernelGGL(k_silu_mul, dim3(blocks_for(I)), dim3(256), 0, st, g, u, I, h);
    AIPU_TRY(hipGetLastError());
    return launch_gemv_ref(type, wd, H, I, h, 1, y, nullptr, st);
}

// The FFN half of decoder_block (tools/glm_model_q4k_ref.py:797-810) around the MoE step:
// nrm = rmsnorm(h, gamma) (:451-465), then the MoE step on nrm with the residual
// y = bf16(h + fbuf) applied to its output (fused into the last down launch on the
// matrix-core path).  a.x is h and a.y the block output; the MoE workspace comes first in
// `a.ws`, then nrm.
int64_t moe_layer_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk) {
    return moe_workspace_bytes(E, H, I, topk) + up(H * 2);
}

hipError_t launch_moe_layer_decode(const MoeArgs& a, const uint16_t* gamma, hipStream_t st) {
    uint16_t* nrm = (uint16_t*)((uint8_t*)a.ws + moe_workspace_bytes(a.E, a.H, a.I, a.topk));
    MoeArgs m = a;
    m.x = nrm;
    m.resid = a.x;
    // fast mode with a Q4_K router on the persistent one-row kernel: the RMSNorm runs in the
    // router's launch (each compute wave's activation pair is one wave of the norm's reduction),
    // with the same bits as the separate norm kernel followed by the router GEMV
    if (a.mode == AIPU_MODE_FAST && a.router_type == T_Q4_K && a.H <= 8192 &&
        ((uintptr_t)a.x | (uintptr_t)gamma | (uintptr_t)nrm) % 16 == 0 && gemv_persist_norm_supported(a.E, a.H)) {
        uint16_t* logits = (uint16_t*)((uint8_t*)a.ws + ws_layout(a.E, a.H, a.I, a.topk).logits);
        AIPU_TRY(launch_gemv_persist_norm((const uint8_t*)a.router_w, a.E, a.H, a.x, gamma, recip_fp32_bits(a.H), nrm,
                                          logits, st));
        m.logits_ready = true;
        return launch_moe_decode(m, st);
    }
    AIPU_TRY(launch_rmsnorm(a.x, gamma, a.H, nrm, a.mode, st));
    return launch_moe_decode(m, st);
}

}  // namespace aipu
