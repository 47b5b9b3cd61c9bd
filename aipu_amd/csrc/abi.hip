// The extern "C" entry points declared in include/aipu_q4k.h: argument validation (before
// any GPU work), dispatch to the launchers, and the thread-local error message.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "common.hpp"
#include "launch.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int ok() {
    g_err.clear();
    return AIPU_OK;
}

int hip_status(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(AIPU_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

bool known_type(int t) {
    return t == aipu::T_Q4_K || t == aipu::T_Q6_K || t == aipu::T_Q8_0 || t == aipu::T_F16 || t == aipu::T_BF16;
}

const char* type_name(int t) {
    switch (t) {
        case aipu::T_Q4_K: return "Q4_K";
        case aipu::T_Q6_K: return "Q6_K";
        case aipu::T_Q8_0: return "Q8_0";
        case aipu::T_F16: return "F16";
        case aipu::T_BF16: return "BF16";
        default: return "?";
    }
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Alignment the kernels need for a weight pointer of this type: Q4_K blocks (both modes)
// and bf16 rows in fast mode are read with 16-B loads, everything else with 2-B loads.
uintptr_t weight_align(int t, int mode = AIPU_MODE_FAST) {
    return (t == aipu::T_Q4_K || (t == aipu::T_BF16 && mode == AIPU_MODE_FAST)) ? 16 : 2;
}

hipStream_t S(void* s) { return (hipStream_t)s; }

// Shared checks for a GEMV-shaped call.  k256: K must be a whole number of 256-weight
// super-blocks (every entry point but the plain GEMV, which serves any multiple of the block).
int check_gemv(int type, const void* w, int64_t N, int64_t K, const void* x, int64_t M, const void* y,
               const void* yf, int mode, bool k256 = true) {
    if (!known_type(type)) return fail(AIPU_ERR_TYPE, "unsupported ggml type %d", type);
    if (!w || !x || !y) return fail(AIPU_ERR_ARG, "null w/x/y pointer");
    if (mode != AIPU_MODE_FAST && mode != AIPU_MODE_REF) return fail(AIPU_ERR_ARG, "mode must be 0 (fast) or 1 (ref)");
    if (N < 1 || K < 1 || M < 1) return fail(AIPU_ERR_SHAPE, "N, K, M must be >= 1 (got %lld, %lld, %lld)",
                                            (long long)N, (long long)K, (long long)M);
    if (K % aipu::type_qk(type))
        return fail(AIPU_ERR_SHAPE, "K=%lld is not a multiple of the %s block size %d", (long long)K, type_name(type),
                    aipu::type_qk(type));
    if (k256 && K % 256) return fail(AIPU_ERR_SHAPE, "K=%lld must be a multiple of 256", (long long)K);
    if (N > (1LL << 31) || M > (1LL << 24)) return fail(AIPU_ERR_SHAPE, "N or M out of range");
    if (!aligned(w, weight_align(type, mode)))
        return fail(AIPU_ERR_ALIGN, "%s weights must be %d-byte aligned", type_name(type),
                    (int)weight_align(type, mode));
    if (!aligned(x, mode == AIPU_MODE_FAST ? 16 : 2))
        return fail(AIPU_ERR_ALIGN, "activations must be %d-byte aligned", mode == AIPU_MODE_FAST ? 16 : 2);
    if (!aligned(y, 2) || (yf && !aligned(yf, 4))) return fail(AIPU_ERR_ALIGN, "misaligned output");
    return AIPU_OK;
}

// Fast kernels exist for every type: Q4_K on the matrix cores, bf16 in the streaming
// kernel, Q6_K / Q8_0 / F16 in the mixed-type kernel (K up to its staging limit).  Larger K,
// and K that is not a whole number of 256-weight super-blocks, are served by the exact
// kernel, whose results trivially satisfy the fast-mode tolerance.
bool has_fast(int type, int64_t K) {
    if (K % 256) return false;   // a partial super-block: the exact kernel
    if (type == aipu::T_Q4_K || type == aipu::T_BF16) return true;
    return aipu::gemv_mixed_supported(type, K);
}

}  // namespace

extern "C" {

int aipu_version(void) { return 200; }

const char* aipu_last_error(void) { return g_err.c_str(); }

int aipu_dequant(int ggml_type, const void* blocks, int64_t n_weights, float* out, void* stream) {
    if (!known_type(ggml_type)) return fail(AIPU_ERR_TYPE, "unsupported ggml type %d", ggml_type);
    if (!blocks || !out) return fail(AIPU_ERR_ARG, "null pointer");
    if (n_weights < 0 || n_weights % aipu::type_qk(ggml_type))
        return fail(AIPU_ERR_SHAPE, "n_weights=%lld is not a whole number of %s blocks", (long long)n_weights,
                    type_name(ggml_type));
    if (!aligned(blocks, ggml_type == aipu::T_Q4_K ? 4 : 2) || !aligned(out, 4))
        return fail(AIPU_ERR_ALIGN, "misaligned blocks or output");
    if (n_weights == 0) return ok();
    return hip_status(aipu::launch_dequant(ggml_type, blocks, n_weights, out, S(stream)), "aipu_dequant");
}

int aipu_q4k_scale_min(const void* blocks, int64_t n_blocks, uint16_t* out, void* stream) {
    if (!blocks || !out) return fail(AIPU_ERR_ARG, "null pointer");
    if (n_blocks < 0) return fail(AIPU_ERR_SHAPE, "negative block count");
    if (!aligned(blocks, 4) || !aligned(out, 2)) return fail(AIPU_ERR_ALIGN, "misaligned blocks or output");
    if (n_blocks == 0) return ok();
    return hip_status(aipu::launch_q4k_scale_min(blocks, n_blocks, out, S(stream)), "aipu_q4k_scale_min");
}

int aipu_bf16_round(const float* x, int64_t n, uint16_t* out, void* stream) {
    if (!x || !out) return fail(AIPU_ERR_ARG, "null pointer");
    if (n < 0) return fail(AIPU_ERR_SHAPE, "negative length");
    if (!aligned(x, 4) || !aligned(out, 2)) return fail(AIPU_ERR_ALIGN, "misaligned input or output");
    if (n == 0) return ok();
    return hip_status(aipu::launch_bf16_round(x, n, out, S(stream)), "aipu_bf16_round");
}

int aipu_gemv_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M, uint16_t* y, float* y_f32,
                  void* stream) {
    if (!w || !x || !y) return fail(AIPU_ERR_ARG, "null w/x/y pointer");
    if (N < 1 || K < 1 || M < 1) return fail(AIPU_ERR_SHAPE, "N, K, M must be >= 1");
    if (!aligned(w, 4) || !aligned(x, 4) || !aligned(y, 2) || (y_f32 && !aligned(y_f32, 4)))
        return fail(AIPU_ERR_ALIGN, "misaligned pointer");
    return hip_status(aipu::launch_gemv_ref_f32(w, N, K, x, M, y, y_f32, S(stream)), "aipu_gemv_f32");
}

int aipu_gemv(int ggml_type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
              float* y_f32, int mode, void* stream) {
    if (mode != AIPU_MODE_FAST && mode != AIPU_MODE_REF && mode != AIPU_MODE_FAST_DENSE)
        return fail(AIPU_ERR_ARG, "mode must be 0 (fast), 1 (ref) or 2 (fast, dense batches)");
    const bool dense = mode == AIPU_MODE_FAST_DENSE;
    if (dense) mode = AIPU_MODE_FAST;   // the same arguments, alignment and kernels but for Q4_K batches
    int rc = check_gemv(ggml_type, w, N, K, x, M, y, y_f32, mode, false);
    if (rc) return rc;
    if (mode == AIPU_MODE_FAST && has_fast(ggml_type, K))
        return hip_status(aipu::launch_gemv_fast(ggml_type, w, N, K, x, M, y, y_f32, S(stream), dense), "aipu_gemv");
    return hip_status(aipu::launch_gemv_ref(ggml_type, w, N, K, x, M, y, y_f32, S(stream)), "aipu_gemv");
}

int aipu_gemv_tiles(const aipu_tile_desc* tiles, int n_tiles, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                    uint16_t* y, float* y_f32, int mode, void* stream) {
    if (!tiles || n_tiles < 1 || n_tiles > AIPU_MAX_TILES)
        return fail(AIPU_ERR_ARG, "need 1..%d tile descriptors", AIPU_MAX_TILES);
    for (int t = 0; t < n_tiles; ++t) {
        const aipu_tile_desc& d = tiles[t];
        if (d.reserved != 0) return fail(AIPU_ERR_ARG, "tile %d: reserved field must be 0", t);
        if (d.row0 < 0 || d.nrows < 1 || d.row0 + d.nrows > N)
            return fail(AIPU_ERR_SHAPE, "tile %d: rows [%lld, %lld) outside [0, %lld)", t, (long long)d.row0,
                        (long long)(d.row0 + d.nrows), (long long)N);
        int rc = check_gemv(d.ggml_type, d.w, d.nrows, K, x, M, y, y_f32, mode);
        if (rc) return fail(rc, "tile %d: %s", t, g_err.c_str());
        for (int u = 0; u < t; ++u) {
            const aipu_tile_desc& e = tiles[u];
            if (d.row0 < e.row0 + e.nrows && e.row0 < d.row0 + d.nrows)
                return fail(AIPU_ERR_SHAPE, "tiles %d and %d overlap", u, t);
        }
    }
    return hip_status(aipu::launch_gemv_tiles(tiles, n_tiles, N, K, x, M, y, y_f32, mode, S(stream)),
                      "aipu_gemv_tiles");
}

int aipu_glm_silu(const uint16_t* x, int64_t n, uint16_t* y, void* stream) {
    if (!x || !y) return fail(AIPU_ERR_ARG, "null pointer");
    if (n < 0) return fail(AIPU_ERR_SHAPE, "negative length");
    if (!aligned(x, 2) || !aligned(y, 2)) return fail(AIPU_ERR_ALIGN, "misaligned pointer");
    if (n == 0) return ok();
    return hip_status(aipu::launch_act(0, x, n, y, S(stream)), "aipu_glm_silu");
}

int aipu_glm_sigmoid(const uint16_t* x, int64_t n, uint16_t* y, void* stream) {
    if (!x || !y) return fail(AIPU_ERR_ARG, "null pointer");
    if (n < 0) return fail(AIPU_ERR_SHAPE, "negative length");
    if (!aligned(x, 2) || !aligned(y, 2)) return fail(AIPU_ERR_ALIGN, "misaligned pointer");
    if (n == 0) return ok();
    return hip_status(aipu::launch_act(1, x, n, y, S(stream)), "aipu_glm_sigmoid");
}

int aipu_fp32_rsqrt(const float* x, int64_t n, float* y, void* stream) {
    if (!x || !y) return fail(AIPU_ERR_ARG, "null pointer");
    if (n < 0) return fail(AIPU_ERR_SHAPE, "negative length");
    if (!aligned(x, 4) || !aligned(y, 4)) return fail(AIPU_ERR_ALIGN, "misaligned pointer");
    if (n == 0) return ok();
    return hip_status(aipu::launch_rsqrt(x, n, y, S(stream)), "aipu_fp32_rsqrt");
}

int aipu_router_topk(const uint16_t* logits, int64_t E, int topk, uint32_t scale_bits, int32_t* sel_idx,
                     uint16_t* sel_w, uint16_t* gates, void* stream) {
    if (!logits || !sel_idx || !sel_w) return fail(AIPU_ERR_ARG, "null pointer");
    if (E < 1 || E > 4096) return fail(AIPU_ERR_SHAPE, "E=%lld outside 1..4096", (long long)E);
    if (topk < 1 || topk > 32 || topk > E) return fail(AIPU_ERR_SHAPE, "topk=%d outside 1..min(32, E)", topk);
    if (!aligned(logits, 2) || !aligned(sel_idx, 4) || !aligned(sel_w, 2) || (gates && !aligned(gates, 2)))
        return fail(AIPU_ERR_ALIGN, "misaligned pointer");
    return hip_status(aipu::launch_router_tail(logits, (int)E, topk, scale_bits, sel_idx, sel_w, gates, S(stream)),
                      "aipu_router_topk");
}

int64_t aipu_moe_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk) {
    if (E < 1 || H < 1 || I < 1 || topk < 1) return -1;
    return aipu::moe_workspace_bytes(E, H, I, topk);
}

int aipu_swiglu_expert(int ggml_type, const void* wg, const void* wu, const void* wd, int64_t H, int64_t I,
                       const uint16_t* x, uint16_t* y, uint16_t* h_out, int mode, void* workspace, int64_t ws_bytes,
                       void* stream) {
    if (!wu || !wd) return fail(AIPU_ERR_ARG, "null weight pointer");
    int rc = check_gemv(ggml_type, wg, I, H, x, 1, y, nullptr, mode);
    if (rc) return rc;
    if (H % 256 || I % 256) return fail(AIPU_ERR_SHAPE, "H and I must be multiples of 256");
    if (!aligned(wu, weight_align(ggml_type, mode)) || !aligned(wd, weight_align(ggml_type, mode)))
        return fail(AIPU_ERR_ALIGN, "misaligned weights");
    if (h_out && !aligned(h_out, 16)) return fail(AIPU_ERR_ALIGN, "h_out must be 16-byte aligned");
    const int64_t need = aipu::moe_workspace_bytes(1, H, I, 1);
    if (!workspace || ws_bytes < need || !aligned(workspace, 256))
        return fail(AIPU_ERR_WORKSPACE, "workspace must be 256-byte aligned and >= %lld bytes", (long long)need);
    if (mode == AIPU_MODE_FAST && ggml_type == aipu::T_Q4_K && I / 256 > 8 * 8)
        return fail(AIPU_ERR_SHAPE, "fast mode supports I <= 16384");
    return hip_status(aipu::launch_swiglu_expert(ggml_type, wg, wu, wd, H, I, x, y, h_out, mode, workspace, S(stream)),
                      "aipu_swiglu_expert");
}

// Checks shared by the MoE decode step and the MoE layer step; fills `a` (need = workspace
// bytes the caller's entry point requires).
static int moe_args(int router_type, const void* router_w, int ggml_type, const void* gate_exps, const void* up_exps,
                    const void* down_exps, const void* shared_gate, const void* shared_up, const void* shared_down,
                    int64_t E, int64_t H, int64_t I, int topk, uint32_t scale_bits, const uint16_t* x, uint16_t* y,
                    int32_t* sel_idx, uint16_t* sel_w, int mode, void* workspace, int64_t ws_bytes, int64_t need,
                    aipu::MoeArgs& a) {
    if (!known_type(router_type)) return fail(AIPU_ERR_TYPE, "unsupported router type %d", router_type);
    if (!router_w || !gate_exps || !up_exps || !down_exps) return fail(AIPU_ERR_ARG, "null weight pointer");
    const bool sh_any = shared_gate || shared_up || shared_down;
    const bool sh_all = shared_gate && shared_up && shared_down;
    if (sh_any && !sh_all) return fail(AIPU_ERR_ARG, "shared expert needs all of gate/up/down (or none)");
    if (E < 1 || E > 4096) return fail(AIPU_ERR_SHAPE, "E=%lld outside 1..4096", (long long)E);
    if (topk < 1 || topk > 32 || topk > E) return fail(AIPU_ERR_SHAPE, "topk=%d outside 1..min(32, E)", topk);
    int rc = check_gemv(router_type, router_w, E, H, x, 1, y, nullptr, mode);
    if (rc) return fail(rc, "router: %s", g_err.c_str());
    rc = check_gemv(ggml_type, gate_exps, I, H, x, 1, y, nullptr, mode);
    if (rc) return fail(rc, "experts: %s", g_err.c_str());
    if (I % 256) return fail(AIPU_ERR_SHAPE, "I must be a multiple of 256");
    const uintptr_t wa = weight_align(ggml_type, mode);
    if (!aligned(up_exps, wa) || !aligned(down_exps, wa) || (sh_all && (!aligned(shared_gate, wa) ||
                                                                        !aligned(shared_up, wa) ||
                                                                        !aligned(shared_down, wa))))
        return fail(AIPU_ERR_ALIGN, "misaligned expert weights");
    if ((sel_idx && !aligned(sel_idx, 4)) || (sel_w && !aligned(sel_w, 2)))
        return fail(AIPU_ERR_ALIGN, "misaligned routing outputs");
    if (!workspace || ws_bytes < need || !aligned(workspace, 256))
        return fail(AIPU_ERR_WORKSPACE, "workspace must be 256-byte aligned and >= %lld bytes", (long long)need);
    if (mode == AIPU_MODE_FAST && ggml_type == aipu::T_Q4_K && I / 256 > 8 * 8)
        return fail(AIPU_ERR_SHAPE, "fast mode supports I <= 16384");
    a.router_type = router_type;
    a.router_w = router_w;
    a.type = ggml_type;
    a.gate_exps = (const uint8_t*)gate_exps;
    a.up_exps = (const uint8_t*)up_exps;
    a.down_exps = (const uint8_t*)down_exps;
    a.sh_gate = (const uint8_t*)shared_gate;
    a.sh_up = (const uint8_t*)shared_up;
    a.sh_down = (const uint8_t*)shared_down;
    a.E = E;
    a.H = H;
    a.I = I;
    a.topk = topk;
    a.scale_bits = scale_bits;
    a.x = x;
    a.y = y;
    a.sel_idx_out = sel_idx;
    a.sel_w_out = sel_w;
    a.mode = mode;
    a.ws = workspace;
    return AIPU_OK;
}

int aipu_moe_swiglu_decode(int router_type, const void* router_w, int ggml_type, const void* gate_exps,
                           const void* up_exps, const void* down_exps, const void* shared_gate, const void* shared_up,
                           const void* shared_down, int64_t E, int64_t H, int64_t I, int topk, uint32_t scale_bits,
                           const uint16_t* x, uint16_t* y, int32_t* sel_idx, uint16_t* sel_w, int mode,
                           void* workspace, int64_t ws_bytes, void* stream) {
    aipu::MoeArgs a;
    const int rc = moe_args(router_type, router_w, ggml_type, gate_exps, up_exps, down_exps, shared_gate, shared_up,
                            shared_down, E, H, I, topk, scale_bits, x, y, sel_idx, sel_w, mode, workspace, ws_bytes,
                            E >= 1 && topk >= 1 ? aipu::moe_workspace_bytes(E, H, I, topk) : 0, a);
    if (rc) return rc;
    return hip_status(aipu::launch_moe_decode(a, S(stream)), "aipu_moe_swiglu_decode");
}

}  // extern "C"

// ------------------------------------------------- MoE decode step without allocation
// For callers that cannot allocate (code under HIP graph capture, tight serving loops,
// harnesses that forbid it): the MoE step's scratch is a file-scope device array, one copy
// per GPU for the life of the process.  In host code `scratch` is only a stand-in symbol;
// its device address comes from hipGetSymbolAddress, taken once per device with that device
// current, and only that address is ever passed to kernels.  Calls on one GPU share the
// array, so calls that can overlap on one GPU race.  Nothing in it needs to start at zero:
// every call writes what it reads (logits, routing, h, the fp32 running sum).
namespace {

constexpr int64_t kScratchBytes = AIPU_NOALLOC_SCRATCH_BYTES;   // per GPU
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of this GPU's scratch array (the stream's device, or the current device for
// the null stream); looked up on the first call on each device.
int scratch_for(hipStream_t st, void** out) {
    int dev = -1;
    hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
    if (e != hipSuccess) return fail(AIPU_ERR_HIP, "scratch: device of the stream: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(AIPU_ERR_ARG, "scratch: device %d out of range", dev);
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            int prev = -1;
            e = hipGetDevice(&prev);
            if (e == hipSuccess && prev != dev) e = hipSetDevice(dev);
            if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            const hipError_t e2 = (prev >= 0 && prev != dev) ? hipSetDevice(prev) : hipSuccess;
            if (e != hipSuccess || !p)
                return fail(AIPU_ERR_HIP, "scratch: hipGetSymbolAddress on device %d: %s", dev,
                            hipGetErrorString(e != hipSuccess ? e : hipErrorInvalidSymbol));
            if (e2 != hipSuccess) return fail(AIPU_ERR_HIP, "scratch: restoring device %d: %s", prev, hipGetErrorString(e2));
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return AIPU_OK;
}

}  // namespace

extern "C" {

int aipu_moe_swiglu_decode_noalloc(int router_type, const void* router_w, int ggml_type, const void* gate_exps,
                                   const void* up_exps, const void* down_exps, const void* shared_gate,
                                   const void* shared_up, const void* shared_down, int64_t E, int64_t H, int64_t I,
                                   int topk, uint32_t scale_bits, const uint16_t* x, uint16_t* y, int32_t* sel_idx,
                                   uint16_t* sel_w, int mode, void* stream) {
    const int64_t need = E >= 1 && topk >= 1 && H >= 1 && I >= 1 ? aipu::moe_workspace_bytes(E, H, I, topk) : 0;
    if (need > kScratchBytes)
        return fail(AIPU_ERR_WORKSPACE, "aipu_moe_swiglu_decode_noalloc: E=%lld H=%lld I=%lld topk=%d needs %lld "
                                        "bytes of scratch, more than the %lld-byte per-GPU array",
                    (long long)E, (long long)H, (long long)I, topk, (long long)need, (long long)kScratchBytes);
    // every argument is checked (with a stand-in for the scratch address, which moe_args only
    // tests for presence and alignment) before anything touches the GPU
    aipu::MoeArgs a;
    int rc = moe_args(router_type, router_w, ggml_type, gate_exps, up_exps, down_exps, shared_gate, shared_up,
                      shared_down, E, H, I, topk, scale_bits, x, y, sel_idx, sel_w, mode, (void*)(uintptr_t)256,
                      kScratchBytes, need, a);
    if (rc) return rc;
    void* ws = nullptr;
    rc = scratch_for(S(stream), &ws);
    if (rc) return rc;
    a.ws = ws;
    return hip_status(aipu::launch_moe_decode(a, S(stream)), "aipu_moe_swiglu_decode_noalloc");
}

int64_t aipu_moe_batched_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk) {
    if (E < 1 || E > 4096 || H < 1 || I < 1 || topk < 1 || topk > 32) return -1;
    return aipu::moe_batched_workspace_bytes(E, H, I, topk);
}

int aipu_moe_swiglu_decode_batched(int router_type, const void* router_w, int ggml_type, const void* gate_exps,
                                   const void* up_exps, const void* down_exps, const void* shared_gate,
                                   const void* shared_up, const void* shared_down, int64_t E, int64_t H, int64_t I,
                                   int topk, uint32_t scale_bits, const uint16_t* x, int64_t M, uint16_t* y,
                                   int32_t* sel_idx, uint16_t* sel_w, int mode, void* workspace, int64_t ws_bytes,
                                   void* stream) {
    if (M < 1 || M > (1LL << 20)) return fail(AIPU_ERR_SHAPE, "M = %lld out of range", (long long)M);
    aipu::MoeArgs a;
    const bool shape_ok = E >= 1 && E <= 4096 && topk >= 1 && topk <= 32;
    const int rc = moe_args(router_type, router_w, ggml_type, gate_exps, up_exps, down_exps, shared_gate, shared_up,
                            shared_down, E, H, I, topk, scale_bits, x, y, sel_idx, sel_w, mode, workspace, ws_bytes,
                            shape_ok ? aipu::moe_batched_workspace_bytes(E, H, I, topk) : 0, a);
    if (rc) return rc;
    return hip_status(aipu::launch_moe_decode_batched(a, M, S(stream)), "aipu_moe_swiglu_decode_batched");
}

int64_t aipu_moe_layer_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk) {
    if (E < 1 || H < 1 || I < 1 || topk < 1) return -1;
    return aipu::moe_layer_workspace_bytes(E, H, I, topk);
}

int aipu_moe_layer_decode(int router_type, const void* router_w, int ggml_type, const void* gate_exps,
                          const void* up_exps, const void* down_exps, const void* shared_gate, const void* shared_up,
                          const void* shared_down, int64_t E, int64_t H, int64_t I, int topk, uint32_t scale_bits,
                          const uint16_t* h, const uint16_t* gamma, uint16_t* y, int32_t* sel_idx, uint16_t* sel_w,
                          int mode, void* workspace, int64_t ws_bytes, void* stream) {
    if (!gamma || !h || !y) return fail(AIPU_ERR_ARG, "null h, gamma or output pointer");
    if (!aligned(gamma, 2)) return fail(AIPU_ERR_ALIGN, "gamma must be 2-byte aligned");
    aipu::MoeArgs a;
    const int rc = moe_args(router_type, router_w, ggml_type, gate_exps, up_exps, down_exps, shared_gate, shared_up,
                            shared_down, E, H, I, topk, scale_bits, h, y, sel_idx, sel_w, mode, workspace, ws_bytes,
                            E >= 1 && topk >= 1 ? aipu::moe_layer_workspace_bytes(E, H, I, topk) : 0, a);
    if (rc) return rc;
    return hip_status(aipu::launch_moe_layer_decode(a, gamma, S(stream)), "aipu_moe_layer_decode");
}

int aipu_measure_gemv(int what, const void* w, int64_t N, int64_t K, const uint16_t* x, void* stream) {
    if (what != AIPU_MEASURE_EMPTY && what != AIPU_MEASURE_COPY) return fail(AIPU_ERR_ARG, "unknown measurement %d", what);
    if (!w || !x) return fail(AIPU_ERR_ARG, "null pointer");
    if (N < 1 || K < 256 || K % 256 || !aipu::gemv_persist_supported(N, K))
        return fail(AIPU_ERR_SHAPE, "N=%lld K=%lld: the M = 1 persistent kernel serves K = 256 .. 8192 (multiples of 256)",
                    (long long)N, (long long)K);
    if (!aligned(w, 16) || !aligned(x, 16)) return fail(AIPU_ERR_ALIGN, "weights and activations must be 16-byte aligned");
    return hip_status(aipu::launch_gemv_persist((const uint8_t*)w, N, K, x, nullptr, nullptr, S(stream),
                                                what == AIPU_MEASURE_COPY ? 1 : 2),
                      "aipu_measure_gemv");
}

int aipu_wait_timeouts(uint32_t* gave_up) {
    if (!gave_up) return fail(AIPU_ERR_ARG, "null pointer");
    uint32_t a = 0, b = 0, c = 0;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = aipu::wait_gave_up_gemv_persist(&a);
    if (e == hipSuccess) e = aipu::wait_gave_up_gemv_persist_m(&b);
    if (e == hipSuccess) e = aipu::wait_gave_up_moe_persist(&c);
    if (e != hipSuccess) return fail(AIPU_ERR_HIP, "aipu_wait_timeouts: %s", hipGetErrorString(e));
    *gave_up = (a | b | c) ? 1u : 0u;
    return ok();
}

int aipu_rmsnorm(const uint16_t* x, const uint16_t* gamma, int64_t n, uint16_t* y, int mode, void* stream) {
    if (!x || !gamma || !y) return fail(AIPU_ERR_ARG, "null pointer");
    if (n < 1 || n > (1LL << 31)) return fail(AIPU_ERR_SHAPE, "n = %lld out of range", (long long)n);
    if (mode != AIPU_MODE_REF && mode != AIPU_MODE_FAST) return fail(AIPU_ERR_ARG, "unknown mode %d", mode);
    if (!aligned(x, 2) || !aligned(gamma, 2) || !aligned(y, 2)) return fail(AIPU_ERR_ALIGN, "misaligned pointer");
    return hip_status(aipu::launch_rmsnorm(x, gamma, n, y, mode, S(stream)), "aipu_rmsnorm");
}


int64_t aipu_gemm_prefill_workspace_bytes(int64_t M, int64_t K) {
    if (M < 1 || K < aipu::QK_K || K % aipu::QK_K || M > (1LL << 31) || K > (1LL << 31)) return -1;
    return aipu::prefill_workspace_bytes(M, K);
}

int aipu_gemm_prefill(int ggml_type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                      float* y_f32, int precision, void* workspace, int64_t ws_bytes, void* stream) {
    if (ggml_type != aipu::T_Q4_K) return fail(AIPU_ERR_TYPE, "prefill supports Q4_K weights");
    int rc = check_gemv(ggml_type, w, N, K, x, M, y, y_f32, AIPU_MODE_FAST);
    if (rc) return rc;
    if (precision != AIPU_PREFILL_CODES) return fail(AIPU_ERR_ARG, "unknown prefill precision %d", precision);
    if (!aligned(x, 16)) return fail(AIPU_ERR_ALIGN, "x must be 16-byte aligned");
    if (M > (1LL << 24) || N > (1LL << 31) || K > (1LL << 24))
        return fail(AIPU_ERR_SHAPE, "prefill shape out of range (M %lld, N %lld, K %lld)", (long long)M, (long long)N,
                    (long long)K);
    if (64 * (K / aipu::QK_K) * 144 >= (1LL << 32)) return fail(AIPU_ERR_SHAPE, "K too large for prefill");
    const int64_t need = aipu::prefill_workspace_bytes(M, K);
    if (!workspace || ws_bytes < need)
        return fail(AIPU_ERR_WORKSPACE, "prefill workspace of %lld bytes needed, %lld given", (long long)need,
                    (long long)ws_bytes);
    if (!aligned(workspace, 256)) return fail(AIPU_ERR_ALIGN, "workspace must be 256-byte aligned");
    return hip_status(aipu::launch_gemm_prefill(ggml_type, w, N, K, x, M, y, y_f32, precision, workspace, S(stream)),
                      "aipu_gemm_prefill");
}

int64_t aipu_lm_head_workspace_bytes(int64_t V) {
    if (V < 1 || V > (1LL << 31)) return -1;
    return aipu::lm_head_workspace_bytes(V);
}

int aipu_lm_head(const uint16_t* w, int64_t V, int64_t K, const uint16_t* x, uint16_t* logits, int32_t* argmax,
                 void* workspace, int64_t ws_bytes, void* stream) {
    if (!w || !x) return fail(AIPU_ERR_ARG, "null weight or activation pointer");
    if (!logits && !argmax) return fail(AIPU_ERR_ARG, "neither logits nor argmax requested");
    if (V < 1 || V > (1LL << 31)) return fail(AIPU_ERR_SHAPE, "V = %lld out of range", (long long)V);
    if (K < 8 || K % 8 || K > (1LL << 24))
        return fail(AIPU_ERR_SHAPE, "K = %lld must be a positive multiple of 8 (at most 2^24)", (long long)K);
    if (!aligned(w, 16) || !aligned(x, 16)) return fail(AIPU_ERR_ALIGN, "w and x must be 16-byte aligned");
    if (logits && !aligned(logits, 2)) return fail(AIPU_ERR_ALIGN, "logits must be 2-byte aligned");
    if (argmax) {
        const int64_t need = aipu::lm_head_workspace_bytes(V);
        if (!workspace || ws_bytes < need)
            return fail(AIPU_ERR_WORKSPACE, "lm_head workspace of %lld bytes needed, %lld given", (long long)need,
                        (long long)ws_bytes);
        if (!aligned(workspace, 256)) return fail(AIPU_ERR_ALIGN, "workspace must be 256-byte aligned");
        if (!aligned(argmax, 4)) return fail(AIPU_ERR_ALIGN, "argmax must be 4-byte aligned");
    }
    return hip_status(aipu::launch_lm_head(w, V, K, x, logits, argmax, workspace, S(stream)), "aipu_lm_head");
}

int aipu_stream_read(const void* p, int64_t bytes, uint32_t* sink, void* stream) {
    if (!p || !sink) return fail(AIPU_ERR_ARG, "null pointer");
    if (bytes < 16 || bytes % 16) return fail(AIPU_ERR_SHAPE, "bytes must be a positive multiple of 16");
    if (!aligned(p, 16) || !aligned(sink, 4)) return fail(AIPU_ERR_ALIGN, "misaligned pointer");
    return hip_status(aipu::launch_stream_read(p, bytes, sink, S(stream)), "aipu_stream_read");
}

}  // extern "C"
