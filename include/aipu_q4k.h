/*
 * aipu_q4k.h -- C ABI of the MI355X (gfx950) Q4_K GEMM core.
 *
 * A drop-in for the numeric entry points of the reference's Python goldens
 * (tools/q4k_ref.py, tools/glm_model_q4k_ref.py).  Every entry point:
 *   - takes plain device pointers and int64 sizes (no framework types);
 *   - is stream-ordered on the hipStream_t passed as `stream` (NULL = default stream)
 *     and never synchronises the host;
 *   - never allocates device memory; entry points that need scratch take a caller-owned
 *     `workspace` (any contents) of at least the size *_workspace_bytes() returns;
 *   - validates its arguments before touching the GPU and returns AIPU_OK (0) or a negative
 *     status; aipu_last_error() then returns a thread-local message.
 *
 * Weights are ggml row blocks: row n (= output n) holds K/QK consecutive blocks
 * (Q4_K 144 B / 256 w, Q6_K 210 B / 256 w, Q8_0 34 B / 32 w, F16 2 B / w, BF16 2 B / w),
 * i.e. the GGUF tensor layout ne = [K, N].  Activations and outputs are bf16 bit patterns,
 * row-major [M][K] and [M][N].
 *
 * mode: AIPU_MODE_REF reproduces the reference's arithmetic bit-for-bit (exact dequant,
 *       sequential fp32 MAC in K order, bf16 RNE; tools/q4k_ref.py:67-92).
 *       AIPU_MODE_FAST is the bandwidth-optimised path: dequantised weights are exact, fp32
 *       accumulators are within 1e-5 * sum|a*w| of exact, bf16 outputs within 1 ulp of
 *       AIPU_MODE_REF.  Both are deterministic (run-to-run bitwise identical).  In both, row m
 *       of a multi-row GEMV is bit-identical to the one-row call on that row (a speculative-
 *       verify batch reproduces greedy decoding, the reference's PE_M gate, Makefile:1488-1508).
 */
#ifndef AIPU_Q4K_H
#define AIPU_Q4K_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (tools/ckpt_pack_q4k.py:58-68 enumerates F16=1, Q8_0=8, Q4_K=12, Q6_K=14;
 * BF16=30 is ggml's id for bf16 weights, used by the bf16 router of BASELINE config 2). */
#define AIPU_TYPE_F16  1
#define AIPU_TYPE_Q8_0 8
#define AIPU_TYPE_Q4_K 12
#define AIPU_TYPE_Q6_K 14
#define AIPU_TYPE_BF16 30

#define AIPU_MODE_FAST       0
#define AIPU_MODE_REF        1
#define AIPU_MODE_FAST_DENSE 2   /* aipu_gemv only: see there */

#define AIPU_OK             0
#define AIPU_ERR_ARG       -1   /* null pointer or bad enum */
#define AIPU_ERR_TYPE      -2   /* unsupported ggml type for this entry point */
#define AIPU_ERR_SHAPE     -3   /* size not a whole number of blocks, or out of range */
#define AIPU_ERR_ALIGN     -4   /* pointer misaligned for the type's loads */
#define AIPU_ERR_HIP       -5   /* a HIP launch failed */
#define AIPU_ERR_WORKSPACE -6   /* workspace missing or too small */

/* Library version (major*10000 + minor*100 + patch) and the thread-local message of the
 * last failing call on this thread. */
int aipu_version(void);
const char* aipu_last_error(void);

/* Exact dequantisation of n_weights (whole blocks) to fp32.
 * Replaces tools/q4k_ref.py:39-65 (dequantize_block_q4_K / dequantize_row_q4_K),
 * tools/q4k_ref.py:105-124 (dequantize_block_q6_K), tools/q4k_ref.py:126-129
 * (dequantize_block_q8_0) and the F16 passthrough tools/glm_model_q4k_ref.py:61-63.
 * Output is bit-identical to the reference. */
int aipu_dequant(int ggml_type, const void* blocks, int64_t n_weights, float* out, void* stream);

/* Q4_K 6-bit scale/min unpack for every sub-block of n_blocks blocks:
 * out[8*b + j] = sc | (m << 8).  Replaces tools/q4k_ref.py:27-37 (get_scale_min_k4). */
int aipu_q4k_scale_min(const void* blocks, int64_t n_blocks, uint16_t* out, void* stream);

/* fp32 -> bf16 RNE (inf/nan truncated).  Replaces tools/q4k_ref.py:76-84 (bf16_round). */
int aipu_bf16_round(const float* x, int64_t n, uint16_t* out, void* stream);

/* Reference-order GEMV on already-dequantised fp32 weights w[N][K] and fp32 activations
 * x[M][K] (bf16-valued in the reference's use): y[m][n] = bf16(sequential fp32
 * sum_k x[m][k]*w[n][k]).  Replaces tools/q4k_ref.py:86-92 (matmul_q4k_col) and
 * tools/glm_model_q4k_ref.py:470-472 (matmul_q4k).  y_f32 nullable. */
int aipu_gemv_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M,
                  uint16_t* y, float* y_f32, void* stream);

/* The GEMM core: y[M][N] = bf16(x[M][K] . dequant(w)^T) straight from ggml blocks.
 * Replaces matmul_q4k(x, QW.dequant()) (tools/glm_model_q4k_ref.py:470-472 with
 * tools/q4k_matmul_gen.py:28-40) and the glm_matmul_q4k datapath (src/glm_matmul_q4k.v:50-288).
 * Types: Q4_K, Q6_K, Q8_0, F16, BF16.  K must be a multiple of the type's block: 256 for
 * Q4_K and Q6_K, 32 for Q8_0 (tools/q4k_ref.py:126-129), 1 for F16 and BF16.  A K that is not
 * a multiple of 256 runs the reference-order kernel in both modes (its results satisfy the
 * fast-mode tolerance).  The other entry points below (tiles, SwiGLU, MoE, prefill) work in
 * 256-weight super-blocks along K for every type, as the reference's datapath does (a Q8_0
 * super-block is 8 blocks of 32; src/glm_matmul_q4k.v:90-91, tools/q4k_mixed_gen.py:131,143,296).
 * y_f32 (nullable) receives the fp32 accumulators.  M >= 1 (M = K+1 <= 8 for speculative
 * verification batches; large M is served too, see aipu_gemm_prefill).  In AIPU_MODE_FAST and
 * AIPU_MODE_REF each row of the result is bit-identical to the one-row call on that row, for
 * every type and shape.  AIPU_MODE_FAST_DENSE is AIPU_MODE_FAST except for Q4_K batches of
 * 2..8 rows at K = 2048, 4096, 6144: those run the dense multi-row kernel, whose rows agree with
 * their one-row results within the fast-mode tolerance only (a row's bits still depend neither
 * on the other rows nor on its position in the batch); for callers that batch independent rows
 * and do not need batch == one-row bits (it is faster from four rows on). */
int aipu_gemv(int ggml_type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
              uint16_t* y, float* y_f32, int mode, void* stream);

/* One tile of a mixed-type weight sequence: rows [row0, row0+nrows) of the output are
 * produced by `w` (nrows ggml rows of the tile's type, all of length K). */
typedef struct aipu_tile_desc {
    int32_t ggml_type;
    int32_t reserved;     /* must be 0 */
    const void* w;
    int64_t row0;
    int64_t nrows;
} aipu_tile_desc;

#define AIPU_MAX_TILES 64

/* Mixed-type GEMV over up to AIPU_MAX_TILES tiles in one launch: the per-column w_type
 * mux of src/glm_matmul_q4k.v:76-101,197-259 and the tile sequence of
 * tools/q4k_mixed_gen.py:382-440.  Tiles must not overlap; rows not covered are left
 * untouched.  N is the total output width. */
int aipu_gemv_tiles(const aipu_tile_desc* tiles, int n_tiles, int64_t N, int64_t K,
                    const uint16_t* x, int64_t M, uint16_t* y, float* y_f32, int mode,
                    void* stream);

/* Bit-exact glm_act activations on bf16 patterns.  Replace
 * tools/glm_model_q4k_ref.py:293-294 (glm_sigmoid) and :296-299 (glm_silu). */
int aipu_glm_silu(const uint16_t* x, int64_t n, uint16_t* y, void* stream);
int aipu_glm_sigmoid(const uint16_t* x, int64_t n, uint16_t* y, void* stream);

/* Bit-exact fp32_rsqrt (magic seed + 2 Newton steps).  Replaces
 * tools/glm_model_q4k_ref.py:96-116. */
int aipu_fp32_rsqrt(const float* x, int64_t n, float* y, void* stream);

/* MoE router tail on E bf16 logits: sigmoid -> top-k by (fp32 desc, index asc) -> balanced
 * fp32 add tree -> rs = rsqrt(s)^2 * scale -> bf16 weights.  Replaces
 * tools/glm_model_q4k_ref.py:669-699 (moe_router after its GEMV).  gates (nullable)
 * receives the E bf16 sigmoid gates.  1 <= topk <= 32 <= ... E <= 4096. */
int aipu_router_topk(const uint16_t* logits, int64_t E, int topk, uint32_t scale_bits,
                     int32_t* sel_idx, uint16_t* sel_w, uint16_t* gates, void* stream);

/* Workspace bytes for aipu_swiglu_expert / aipu_moe_swiglu_decode.  The workspace holds the
 * router logits, the routing decision, h and per-slot scratch; every call writes what it
 * reads, so its contents on entry do not matter.  It must not be shared by calls that can
 * run concurrently.  Once an aipu_moe_swiglu_decode or aipu_moe_layer_decode call has run on
 * its stream, the workspace can be inspected: bytes [0, 2E) hold the step's router logits
 * (E bf16, the ones it routed from), and from byte 256 * ceil(E / 128) + 512 the SwiGLU
 * activations h of every slot (I bf16 per slot, in slot order, the shared expert last). */
int64_t aipu_moe_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk);

/* One SwiGLU expert: gate/up GEMVs (bf16), h = bf16(f32(silu(gate)) * f32(up)),
 * y = bf16 GEMV(h, down).  Replaces tools/glm_model_q4k_ref.py:702-708 (swiglu_expert)
 * and src/swiglu_expert_q4k.v:22-217.  wg/wu: [I][H/QK] blocks, wd: [H][I/QK] blocks.
 * h_out (nullable) receives h[I].  Workspace: aipu_moe_workspace_bytes(1, H, I, 1). */
int aipu_swiglu_expert(int ggml_type, const void* wg, const void* wu, const void* wd,
                       int64_t H, int64_t I, const uint16_t* x, uint16_t* y, uint16_t* h_out,
                       int mode, void* workspace, int64_t ws_bytes, void* stream);

/* One MoE FFN decode step (M = 1): router GEMV (router_type BF16 or any ggml type,
 * router_w [E][H]) -> router tail -> for each selected expert in slot order a SwiGLU
 * expert from the ggml `_exps` stacks gate/up [E][I][H/QK], down [E][H][I/QK] ->
 * slot-ordered fp32 combine facc += f32(g*y_e), + optional shared expert (weight 1)
 * -> bf16 y[H].  Replaces the MoE half of tools/glm_model_q4k_ref.py:797-809
 * (decoder_block) with moe_router :663-681 and swiglu_expert :702-708; RTL
 * src/glm_decoder_block_q4k.v:494-497,636-650.  shared_* may all be NULL.
 * sel_idx[topk] / sel_w[topk] (nullable) receive the routing decision. */
int aipu_moe_swiglu_decode(int router_type, const void* router_w, int ggml_type,
                           const void* gate_exps, const void* up_exps, const void* down_exps,
                           const void* shared_gate, const void* shared_up,
                           const void* shared_down, int64_t E, int64_t H, int64_t I, int topk,
                           uint32_t scale_bits, const uint16_t* x, uint16_t* y,
                           int32_t* sel_idx, uint16_t* sel_w, int mode, void* workspace,
                           int64_t ws_bytes, void* stream);

/* aipu_moe_swiglu_decode without a workspace argument and without any allocation: no
 * counterpart in the reference.  It is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid allocation).  The
 * step's scratch is a library-owned per-GPU device array of AIPU_NOALLOC_SCRATCH_BYTES, held
 * from the first call on a GPU until the process ends; shapes whose
 * aipu_moe_workspace_bytes() exceeds it return AIPU_ERR_WORKSPACE.  All calls on one GPU
 * share that array, so calls that can overlap on one GPU (several streams or host threads)
 * race: serialise them.  Results are bit-identical to aipu_moe_swiglu_decode. */
#define AIPU_NOALLOC_SCRATCH_BYTES (4LL << 20)
int aipu_moe_swiglu_decode_noalloc(int router_type, const void* router_w, int ggml_type,
                                   const void* gate_exps, const void* up_exps,
                                   const void* down_exps, const void* shared_gate,
                                   const void* shared_up, const void* shared_down, int64_t E,
                                   int64_t H, int64_t I, int topk, uint32_t scale_bits,
                                   const uint16_t* x, uint16_t* y, int32_t* sel_idx,
                                   uint16_t* sel_w, int mode, void* stream);

/* MoE decode step for M activation rows x[M][H] -> y[M][H], routing per row
 * (sel_idx[M][topk], sel_w[M][topk], nullable, in each row's router order).  M = 1 is
 * aipu_moe_swiglu_decode (routed experts combined in slot order).  M > 1 follows the
 * union-skip batch of src/glm_decoder_block_q4k.v:530-560,836-906: the union of the rows'
 * experts is evaluated once, in ascending expert index, and each row accumulates
 * facc += f32(gate * bf16(y_e)) for its own experts in that order, then the shared expert
 * with weight 1.  Workspace: aipu_moe_batched_workspace_bytes(E, H, I, topk) bytes, any
 * contents; other arguments as aipu_moe_swiglu_decode. */
int64_t aipu_moe_batched_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk);
int aipu_moe_swiglu_decode_batched(int router_type, const void* router_w, int ggml_type,
                                   const void* gate_exps, const void* up_exps, const void* down_exps,
                                   const void* shared_gate, const void* shared_up,
                                   const void* shared_down, int64_t E, int64_t H, int64_t I,
                                   int topk, uint32_t scale_bits, const uint16_t* x, int64_t M,
                                   uint16_t* y, int32_t* sel_idx, uint16_t* sel_w, int mode,
                                   void* workspace, int64_t ws_bytes, void* stream);

/* RMSNorm of one bf16 vector: inv = fp32_rsqrt(f32(f32(sumsq * recip_fp32(n)) + 1e-5)),
 * y[i] = bf16(f32(f32(x[i] * inv) * gamma[i])).  Replaces rmsnorm
 * (tools/glm_model_q4k_ref.py:451-465, recip_fp32 :434-449; RTL src/rmsnorm_unit.v).
 * AIPU_MODE_REF sums the squares in element order (bit-exact); AIPU_MODE_FAST sums them as a
 * tree (tolerance mode). */
int aipu_rmsnorm(const uint16_t* x, const uint16_t* gamma, int64_t n, uint16_t* y, int mode,
                 void* stream);

/* The FFN half of one MoE decoder block: y = bf16(f32(h) + f32(fbuf)), fbuf = the MoE decode
 * step (as aipu_moe_swiglu_decode) on rmsnorm(h, gamma).  Replaces
 * tools/glm_model_q4k_ref.py:797-810 (decoder_block after the attention residual).
 * Arguments as aipu_moe_swiglu_decode with x -> h and gamma[H] added; the workspace is
 * aipu_moe_layer_workspace_bytes(E, H, I, topk) bytes, any contents.  In AIPU_MODE_FAST the
 * output equals aipu_rmsnorm (fast) followed by aipu_moe_swiglu_decode and the residual, bit for
 * bit; with a Q4_K router, H <= 8192 and 16-B aligned h and gamma the norm runs inside the
 * router's launch. */
int64_t aipu_moe_layer_workspace_bytes(int64_t E, int64_t H, int64_t I, int topk);
int aipu_moe_layer_decode(int router_type, const void* router_w, int ggml_type,
                          const void* gate_exps, const void* up_exps, const void* down_exps,
                          const void* shared_gate, const void* shared_up,
                          const void* shared_down, int64_t E, int64_t H, int64_t I, int topk,
                          uint32_t scale_bits, const uint16_t* h, const uint16_t* gamma,
                          uint16_t* y, int32_t* sel_idx, uint16_t* sel_w, int mode,
                          void* workspace, int64_t ws_bytes, void* stream);

/* Prefill GEMM for large M on the matrix cores: y[M][N] = bf16(x[M][K] . dequant(w)^T),
 * tolerance mode (|acc - exact| <= 1e-5 * sum|a*w|; the summation order differs from the
 * reference, use aipu_gemv(..., AIPU_MODE_REF) for the bit-exact order).  Types: Q4_K.
 * y_f32 (nullable) receives the fp32 accumulators [M][N].
 * precision must be AIPU_PREFILL_CODES: the products a * (sc*q) run on fp16 matrix-core
 * instructions with exact integer codes sc*q and each activation row scaled by a power of
 * two into fp16 range, the min term on bf16 instructions with exactly split sub-block sums,
 * and d / dmin are applied in fp32 per super-block.  workspace: caller-owned device memory
 * of at least aipu_gemm_prefill_workspace_bytes(M, K) bytes, 256-B aligned (any contents;
 * it holds the staged activations).  x must be 16-B aligned.  No counterpart in the
 * reference beyond M independent matmul_q4k_col rows (tools/q4k_ref.py:86-92). */
#define AIPU_PREFILL_CODES 0
int64_t aipu_gemm_prefill_workspace_bytes(int64_t M, int64_t K);
int aipu_gemm_prefill(int ggml_type, const void* w, int64_t N, int64_t K, const uint16_t* x,
                      int64_t M, uint16_t* y, float* y_f32, int precision, void* workspace,
                      int64_t ws_bytes, void* stream);

/* bf16 LM head + greedy argmax, bit-exact in the reference's order.  Replaces the LM head
 * of model_forward (tools/glm_model_q4k_ref.py:826-834): logits[v] = matmul_bf16_dot(x,
 * W[v]) (:476-486; products into 7 round-robin fp32 partial sums in k order, added as
 * ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+0)), bf16 out) and the strict-greater bf16_gt scan
 * from -inf with lower-index ties (:138-148).  w: V rows of K bf16 (row-major, 16-B
 * aligned; GGUF ne = [K, V]); x: K bf16 (16-B aligned); K a multiple of 8.  logits (V bf16)
 * and argmax (one int32) may each be NULL, not both; the argmax needs a workspace of
 * aipu_lm_head_workspace_bytes(V) bytes, 256-B aligned, any contents. */
int64_t aipu_lm_head_workspace_bytes(int64_t V);
int aipu_lm_head(const uint16_t* w, int64_t V, int64_t K, const uint16_t* x, uint16_t* logits,
                 int32_t* argmax, void* workspace, int64_t ws_bytes, void* stream);

/* Health check with no counterpart in the reference.  The persistent kernels (the M = 1 and
 * multi-row GEMVs, the MoE expert legs) coordinate their waves through bounded waits: a wave
 * that waited about 2^22 polls for a post that never came stops waiting rather than hang, and
 * its launch's result is then wrong.  Such a give-up sets a per-device word; this call
 * synchronises the current device, stores 1 in *gave_up if any wait gave up since the last
 * call (0 otherwise) and clears the word. */
int aipu_wait_timeouts(uint32_t* gave_up);

/* Measurement utility with no counterpart in the reference: streams `bytes` (a multiple of
 * 16) from `p` with the same 16-B global loads the GEMV kernels use and folds them into
 * sink[0..255]; used to measure the achievable HBM read ceiling beside the 8 TB/s peak. */
int aipu_stream_read(const void* p, int64_t bytes, uint32_t* sink, void* stream);

/* Measurement utility with no counterpart in the reference: the floors of the M = 1 Q4_K GEMV
 * kernel at one shape (Q4_K weights w[N][K/256], K a multiple of 256 up to 8192, x as for
 * aipu_gemv).  what = AIPU_MEASURE_EMPTY launches an empty kernel with the launch shape (grid,
 * block, LDS) that aipu_gemv uses for this shape at M = 1 and touches no memory;
 * what = AIPU_MEASURE_COPY runs that kernel's weight-copy schedule alone (every weight byte
 * streamed into LDS as the GEMV streams it, nothing computed, nothing written). */
#define AIPU_MEASURE_EMPTY 0
#define AIPU_MEASURE_COPY  1
int aipu_measure_gemv(int what, const void* w, int64_t N, int64_t K, const uint16_t* x, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AIPU_Q4K_H */
