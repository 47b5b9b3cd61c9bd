// Host-side launchers implemented by the kernel translation units; the C ABI (abi.hip)
// validates arguments and calls these.  Every launcher enqueues on `st` and returns the
// hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "aipu_q4k.h"

namespace aipu {

// elementwise.hip
hipError_t launch_dequant(int type, const void* blocks, int64_t n_weights, float* out, hipStream_t st);
hipError_t launch_q4k_scale_min(const void* blocks, int64_t n_blocks, uint16_t* out, hipStream_t st);
hipError_t launch_bf16_round(const float* x, int64_t n, uint16_t* out, hipStream_t st);
hipError_t launch_act(int which, const uint16_t* x, int64_t n, uint16_t* y, hipStream_t st);  // 0 silu, 1 sigmoid
hipError_t launch_rsqrt(const float* x, int64_t n, float* y, hipStream_t st);
hipError_t launch_stream_read(const void* p, int64_t bytes, uint32_t* sink, hipStream_t st);

// router.hip
// Router tail (one wave): routing of E bf16 logits; sel2/selw2 (nullable) receive a copy.
hipError_t launch_router_tail(const uint16_t* logits, int E, int topk, uint32_t scale_bits, int32_t* sel_idx,
                              uint16_t* sel_w, uint16_t* gates, hipStream_t st, int32_t* sel2 = nullptr,
                              uint16_t* selw2 = nullptr);
// bf16 router GEMV: logits[e] = bf16(W[e] . x), one workgroup per expert.
hipError_t launch_router_bf16_logits(const uint16_t* W, const uint16_t* x, int64_t K, int E, uint16_t* logits,
                                     hipStream_t st);
// The same for M <= 8 rows x[M][K] -> logits[M][E] (router rows read once).
hipError_t launch_router_bf16_logits_rows(const uint16_t* W, const uint16_t* x, int64_t K, int E, int M,
                                          uint16_t* logits, hipStream_t st);

// gemv_ref.hip -- bit-exact reference order
hipError_t launch_gemv_ref(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                           uint16_t* y, float* y_f32, hipStream_t st);
// Slot-gathered form (MoE reference path): grid z = slot; slot z < topk uses weight matrix
// sel[z] of the stack (stride wstride bytes), slot topk the shared matrix w_alt.
hipError_t launch_gemv_ref_gather(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                                  uint16_t* y, float* y_f32, int nslots, const int32_t* sel, int topk, int64_t E,
                                  int64_t wstride, const void* w_alt, int64_t x_zstride, int64_t y_zstride,
                                  hipStream_t st);
hipError_t launch_gemv_ref_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M,
                               uint16_t* y, float* y_f32, hipStream_t st);

// gemv_fast.hip -- tolerance-mode streaming GEMV
hipError_t launch_gemv_fast(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                            uint16_t* y, float* y_f32, hipStream_t st, bool dense = false);
hipError_t launch_gemv_tiles(const aipu_tile_desc* tiles, int n_tiles, int64_t N, int64_t K, const uint16_t* x,
                             int64_t M, uint16_t* y, float* y_f32, int mode, hipStream_t st);

// gemv_mixed.hip -- one-launch GEMV over tiles of Q4_K / Q6_K / Q8_0 / F16 / BF16 rows
// (tolerance mode, up to four activation rows per weight pass; row m of y at y + m * ys)
bool gemv_mixed_supported(int type, int64_t K);
hipError_t launch_gemv_mixed(const aipu_tile_desc* tiles, int n_tiles, int64_t K, const uint16_t* x, int64_t M,
                             uint16_t* y, float* y_f32, int64_t ys, hipStream_t st);

// gemv_persist.hip -- persistent single-row Q4_K GEMV (tolerance mode, K <= 8192)
bool gemv_persist_supported(int64_t N, int64_t K);
hipError_t launch_gemv_persist(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, uint16_t* y, float* yf,
                               hipStream_t st, int variant = 0);
// The same with the fast RMSNorm of x in front (norm.hpp's order): y = (rmsnorm(x, gamma)) . W^T,
// and x_norm receives the normalised x (bit-identical to launch_rmsnorm's fast mode followed by
// the GEMV).  x, gamma and x_norm 16-B aligned; at most two 8-row tiles per CU.
bool gemv_persist_norm_supported(int64_t N, int64_t K);
// Two activation rows (x row stride K, y row stride ys) in one launch of the same kernel, each
// row bit-identical to its one-row launch (K <= 6144, at most four 8-row tiles per CU).
bool gemv_persist2_supported(int64_t N, int64_t K);
hipError_t launch_gemv_persist2(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, uint16_t* y, float* yf,
                                int64_t ys, hipStream_t st);
hipError_t launch_gemv_persist_norm(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, const uint16_t* gamma,
                                    uint32_t inv_len_bits, uint16_t* x_norm, uint16_t* y, hipStream_t st);

// gemv_persist_m.hip -- persistent Q4_K GEMV for 2 .. 8 activation rows (tolerance mode,
// K = 2048, 4096, 6144, at most three 8-row tiles per CU).  dense = false: row m is
// bit-identical to the single-row kernels; dense = true: a row agrees with them within the
// tolerance (and does not depend on the other rows of the batch)
bool gemv_persist_m_supported(int64_t N, int64_t K, int64_t M, bool dense);
hipError_t launch_gemv_persist_m(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                                 float* yf, int64_t ys, bool dense, hipStream_t st);

// Persistent kernels (gemv_persist.hip, gemv_persist_m.hip, moe_persist.hip): whether one of
// their bounded waits gave up since the last call (the word is then cleared).
hipError_t wait_gave_up_gemv_persist(uint32_t* flag);
hipError_t wait_gave_up_gemv_persist_m(uint32_t* flag);
hipError_t wait_gave_up_moe_persist(uint32_t* flag);

// gemv_mfma.hip -- matrix-core Q4_K GEMV (tolerance mode).  dense = false: every row of a
// batch is bit-identical to the one-row launch on that row; dense = true allows the dense
// multi-row kernel (rows within the tolerance of their one-row results)
bool gemv_mfma_supported(int64_t N, int64_t K, int64_t M);
hipError_t launch_gemv_mfma(const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                            float* y_f32, int64_t ystride, hipStream_t st, bool dense = false);
bool moe_mfma_supported(int nslots, int64_t H, int64_t I);
// Routing source of the gate/up leg: either `sel` (expert ids already decided) or, when
// `logits` is set, the kernel routes from the logits itself and workgroup 0 publishes the
// decision to sel_pub/selw_pub (and the optional API copies sel_api/selw_api).
struct MoeRoute {
    const int32_t* sel;
    const uint16_t* logits;
    uint32_t scale_bits;
    int32_t* sel_pub;
    uint16_t* selw_pub;
    int32_t* sel_api;
    uint16_t* selw_api;
};
bool moe_route_in_kernel(int64_t E, int topk, int64_t H);
hipError_t launch_moe_gateup_mfma(const uint8_t* G, const uint8_t* U, const uint8_t* shG, const uint8_t* shU,
                                  const MoeRoute& route, int topk, int nslots, int64_t E, int64_t H, int64_t I,
                                  const uint16_t* x, uint16_t* h, hipStream_t st);
// More slots than one workgroup holds (top-8 + shared) run as two launches that hand the
// fp32 running sum over through acc_scratch (H floats); resid (nullable) is added to the
// bf16 result (y = bf16(resid + bf16(facc))).
hipError_t launch_moe_down_mfma(const uint8_t* D, const uint8_t* shD, const int32_t* sel, const uint16_t* selw,
                                int topk, int nslots, int64_t E, int64_t H, int64_t I, const uint16_t* h, uint16_t* y,
                                int passthrough, hipStream_t st, float* acc_scratch = nullptr,
                                const uint16_t* resid = nullptr);

// Persistent expert legs of the single-row step (topk <= 8 routed slots, nslots = topk or
// topk + 1 with the shared expert last, H = 2048 R with R <= 3, I = 2048): gate/up routes from
// route.logits in every workgroup.
bool moe_persist_supported(int64_t E, int topk, int nslots, int64_t H, int64_t I);
hipError_t launch_moe_gateup_persist(const uint8_t* G, const uint8_t* U, const uint8_t* shG, const uint8_t* shU,
                                     const uint8_t* D, const uint8_t* shD, const MoeRoute& route, int topk, int nslots,
                                     int64_t E, int64_t H, int64_t I, const uint16_t* x, uint16_t* h, hipStream_t st);
hipError_t launch_moe_down_persist(const uint8_t* D, const uint8_t* shD, const int32_t* sel, const uint16_t* selw,
                                   int topk, int nslots, int64_t E, int64_t H, int64_t I, const uint16_t* h,
                                   uint16_t* y, const uint16_t* resid, hipStream_t st);

// Batched MoE (M = 2..8 rows) over the union of the rows' experts, matrix-core GEMVs.
// uidx/nslots come from the union pass; after_gateup enqueues h = bf16(silu(g) * u).
struct MoeUnionArgs {
    const uint8_t *G, *U, *D, *shG, *shU, *shD;
    const int32_t* uidx;
    const int32_t* nslots;
    int max_slots, M;
    int64_t H, I;
    const uint16_t* x;   // [M][H]
    uint16_t* gu;        // [slot][2][M][I]
    uint16_t* h;         // [slot][M][I]
    uint16_t* y;         // [slot][M][H]
    hipError_t (*after_gateup_fn)(const MoeUnionArgs&, hipStream_t);
    hipError_t after_gateup(hipStream_t st) const { return after_gateup_fn(*this, st); }
};
bool moe_union_supported(int64_t H, int64_t I, int M);
// Rows per union pass: two when both legs fit the small-batch kernel (weights copied to LDS,
// gate and up of a tile in one workgroup with the SwiGLU fused), else eight.
int moe_union_pass_rows(int64_t H, int64_t I);
hipError_t launch_moe_union_mfma(const MoeUnionArgs& a, hipStream_t st);
hipError_t launch_router_tail_rows(const uint16_t* logits, int M, int E, int topk, uint32_t scale_bits, int32_t* sel,
                                   uint16_t* selw, int32_t* sel2, uint16_t* selw2, hipStream_t st);

// moe.hip
struct MoeArgs {
    int router_type;
    const void* router_w;
    int type;
    const uint8_t* gate_exps;
    const uint8_t* up_exps;
    const uint8_t* down_exps;
    const uint8_t* sh_gate;
    const uint8_t* sh_up;
    const uint8_t* sh_down;
    int64_t E, H, I;
    int topk;
    uint32_t scale_bits;
    const uint16_t* x;
    uint16_t* y;
    int32_t* sel_idx_out;
    uint16_t* sel_w_out;
    int mode;
    void* ws;
    const uint16_t* resid = nullptr;   // when set, y = bf16(resid + bf16(combine)) (block residual)
    bool ascending = false;            // combine the routed experts in ascending expert index
    bool logits_ready = false;         // fast mode: the router logits are already in the workspace
};
int64_t moe_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk);
hipError_t launch_moe_decode(const MoeArgs& a, hipStream_t st);
hipError_t launch_swiglu_expert(int type, const void* wg, const void* wu, const void* wd, int64_t H, int64_t I,
                                const uint16_t* x, uint16_t* y, uint16_t* h_out, int mode, void* ws,
                                hipStream_t st);

// prefill.hip -- matrix-core prefill GEMM (tolerance mode); ws holds prefill_workspace_bytes(M, K)
int64_t prefill_workspace_bytes(int64_t M, int64_t K);
hipError_t launch_gemm_prefill(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                               uint16_t* y, float* y_f32, int precision, void* ws, hipStream_t st);

// lmhead.hip -- bf16 LM head in the reference's 7-way interleaved order, plus argmax;
// ws holds lm_head_workspace_bytes(V) (used only when argmax is requested).
int64_t lm_head_workspace_bytes(int64_t V);
hipError_t launch_lm_head(const void* w, int64_t V, int64_t K, const uint16_t* x, uint16_t* logits, int32_t* argmax,
                          void* ws, hipStream_t st);

// norm.hip -- pre-FFN RMSNorm (mode REF: element-order sum, bit-exact; FAST: tree) and
// the residual add out = bf16(h + f)
uint32_t recip_fp32_bits(int64_t n);
hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* gamma, int64_t n, uint16_t* y, int mode,
                          hipStream_t st);
hipError_t launch_residual_add(const uint16_t* h, const uint16_t* f, int64_t n, uint16_t* out, hipStream_t st);

// moe.hip -- FFN half of a decoder block: y = bf16(h + moe(rmsnorm(h, gamma)))
int64_t moe_layer_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk);
hipError_t launch_moe_layer_decode(const MoeArgs& a, const uint16_t* gamma, hipStream_t st);

// moe_batched.hip -- MoE decode step for M rows: M = 1 is the single-row step (slot-order
// combine); M > 1 evaluates the union of the rows' experts once, each row accumulating its
// own experts in ascending expert index (PE_M > 1 union-skip of the reference RTL).
int64_t moe_batched_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk);
hipError_t launch_moe_decode_batched(const MoeArgs& a, int64_t M, hipStream_t st);

int device_cu_count();

}  // namespace aipu
