// bf16 LM-head GEMV + argmax for gfx950, in the reference's own summation order (bit-exact).
//
// logits[v] = matmul_bf16_dot(x, W[v]) (tools/glm_model_q4k_ref.py:476-486): the products
// x[k] * W[v][k] (one fp32 multiply each) go round-robin into seven fp32 partial sums
// ps[k % 7] in increasing k, and the seven are added as ((ps0 + ps1) + (ps2 + ps3)) +
// ((ps4 + ps5) + (ps6 + 0)), then rounded to bf16.  argmax is the strict-greater bf16
// compare of model_forward (:826-834, bf16_gt :138-148) scanning v upwards from -inf, so
// ties go to the lower index and an all -inf (or -nan) vocabulary gives 0.
//
// Mapping.  Lane = vocabulary row: one wave owns 64 rows and carries each row's seven
// partial sums in registers, so the reference order costs nothing -- every lane walks its
// own row in k order.  The rows stream through LDS in chunks of 224 bf16 (448 B per row, a
// multiple of 7 so every chunk starts on partial sum 0): 29 direct-to-LDS copies per chunk
// fill 64 rows x 29 units of 16 B (28 data units and one pad unit per row, so the 464-B
// pitch puts eight consecutive rows on disjoint LDS banks), and each lane reads its row
// back in groups of seven 16-B units.  Two stages per wave keep one chunk in flight while
// the other is summed.  The chunk length is set by HBM, not by the arithmetic: each chunk
// is 64 separate 448-B row segments 12 KB apart, and shorter segments (112 B) ran at half
// the bandwidth; 448 B is the longest that still lets two waves share a CU's LDS.
//
// x is wave-uniform: its values are read with scalar loads and widened to fp32 there.
// Per output the kernel writes the bf16 logit, and each wave writes its best
// (key, -index) pair; a one-workgroup pass reduces those to the argmax.
#include "launch.hpp"
#include "mfma_gemv.hpp"

namespace aipu {
namespace lm {

constexpr int kL = 7;                      // partial sums (FP_MAC_LAT of the reference pipe)
constexpr int kRows = 64;                  // rows per wave, lane = row
constexpr int kU = 28;                     // 16-B units per row per chunk (a multiple of 7)
constexpr int kS = 2;                      // LDS stages per wave

// Row pitch in LDS: an odd number of 16-B units, so that eight consecutive rows read at the
// same unit start on eight different 4-bank groups; the pad unit is filled without a memory
// access.
__host__ __device__ constexpr int pitch_units(int u) { return u | 1; }

// Order key of a bf16 pattern under bf16_gt: sign-magnitude, +0 == -0.
__device__ __forceinline__ uint32_t bf16_key(uint32_t b) {
    const uint32_t m = b & 0x7FFFu;
    return (b & 0x8000u) ? 0x8000u - m : 0x8000u + m;
}

// The starting candidate of the reference scan: -inf at index 0.
constexpr uint64_t kSentinel = ((uint64_t)(0x8000u - 0x7F80u) << 32) | 0xFFFFFFFFull;

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Seven units (56 bf16, a multiple of 7, so element e of the group feeds ps[e % 7]) of this
// lane's row against the matching 56 activations xs (wave-uniform, scalar loads).
__device__ __forceinline__ void group_sum(const uint8_t* row, const uint32_t* __restrict__ xs, int nu,
                                          float (&ps)[kL]) {
    uint4 v[7];
#pragma unroll
    for (int u = 0; u < 7; ++u)
        if (u < nu) v[u] = *reinterpret_cast<const uint4*>(row + 16 * u);
#pragma unroll
    for (int u = 0; u < 7; ++u) {
        if (u >= nu) break;
        const uint32_t wd[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int e = 8 * u + 2 * h;          // element index within the group
            const uint32_t xw = xs[e >> 1];       // x[e] (low half), x[e + 1] (high half)
            const float x0 = __uint_as_float(xw << 16);
            const float x1 = __uint_as_float(xw & 0xFFFF0000u);
            const float w0 = __uint_as_float(wd[h] << 16);
            const float w1 = __uint_as_float(wd[h] & 0xFFFF0000u);
            ps[e % kL] = ps[e % kL] + x0 * w0;
            ps[(e + 1) % kL] = ps[(e + 1) % kL] + x1 * w1;
        }
    }
}

// One chunk of U units (nu of them valid) of this lane's row, in k order.
template <int U>
__device__ __forceinline__ void chunk_sum(const uint8_t* row, const uint32_t* __restrict__ xs, int nu,
                                          float (&ps)[kL]) {
#pragma unroll
    for (int g = 0; g < U / 7; ++g) {
        if (7 * g >= nu) break;
        group_sum(row + 112 * g, xs + 28 * g, nu - 7 * g < 7 ? nu - 7 * g : 7, ps);
        __builtin_amdgcn_sched_barrier(0);   // one group's activations live in SGPRs at a time
    }
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;

// s_waitcnt immediate for vmcnt(n), n < 64 (gfx9: vmcnt bits 3:0 and 15:14).
__host__ __device__ constexpr int wait_vm(int n) { return (mg::kWaitVm0 & ~0xC00F) | (n & 0x0F) | ((n >> 4) << 14); }

// Issue the P copies of chunk `ch` into one stage (all lanes read zeros without a memory
// access when ch is past the end: the offset lands outside the buffer).
template <int P>
__device__ __forceinline__ void chunk_copy(__amdgpu_buffer_rsrc_t rs, lds_u8* stage, const uint32_t* voff, int ch,
                                           int nch, uint32_t chunk_bytes) {
    const uint32_t soff = ch < nch ? (uint32_t)ch * chunk_bytes : mg::kOOB;
#pragma unroll
    for (int c = 0; c < P; ++c)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(stage + 1024 * c), 16,
                                                 voff[c], soff, 0, mg::kNT);
}

// Copy, wait and sum one stage; the copy of chunk ch + S into the same stage goes out as
// soon as the stage has been read into registers.
template <int U, int S>
__device__ __forceinline__ void stage_step(__amdgpu_buffer_rsrc_t rs, lds_u8* dst, const uint8_t* row,
                                           const uint32_t* voff, const uint32_t* xw, int ch,
                                           int nch, float (&ps)[kL]) {
    constexpr int P = pitch_units(U);
    __builtin_amdgcn_s_waitcnt(wait_vm((S - 1) * P));
    chunk_sum<U>(row, xw + (int64_t)ch * (4 * U), U, ps);
    __builtin_amdgcn_s_waitcnt(mg::kWaitLgkm0);
    chunk_copy<P>(rs, dst, voff, ch + S, nch, 16u * U);
    __builtin_amdgcn_sched_barrier(0);
}

template <int U, int S>
__global__ void __launch_bounds__(64) k_lmhead(const uint8_t* __restrict__ W, int64_t V, int64_t K,
                                               const uint16_t* __restrict__ x, uint16_t* __restrict__ logits,
                                               uint64_t* __restrict__ part) {
    static_assert(U % 7 == 0 && (S == 2 || S == 3), "chunk of whole 7-unit groups, 2 or 3 stages");
    constexpr int P = pitch_units(U);
    static_assert((S - 1) * P < 64, "outstanding copies fit the vmcnt counter");
    constexpr int kSB = kRows * P * 16;
    __shared__ __attribute__((aligned(16))) uint8_t s0[kSB];
    __shared__ __attribute__((aligned(16))) uint8_t s1[kSB];
    __shared__ __attribute__((aligned(16))) uint8_t s2[S > 2 ? kSB : 16];
    const int lane = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * kRows;
    const int64_t nrows = V - row0 < kRows ? V - row0 : kRows;
    const uint32_t rb = (uint32_t)(K * 2);                 // bytes per row
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(W + row0 * (int64_t)rb, (uint32_t)nrows * rb);

    // Copy c, lane l fills LDS unit p = 64c + l = P r + u: row r, unit u of the chunk (the
    // pad unit u = U, if any, reads nothing).
    uint32_t voff[P];
#pragma unroll
    for (int c = 0; c < P; ++c) {
        const int p = 64 * c + lane;
        const int u = p % P;
        voff[c] = u < U ? (uint32_t)(p / P) * rb + 16u * (uint32_t)u : mg::kOOB;
    }

    const int nfull = (int)(K / (8 * U));
    const int tail_units = (int)((K % (8 * U)) / 8);
    const int nch = nfull + (tail_units ? 1 : 0);
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);

    float ps[kL];
#pragma unroll
    for (int j = 0; j < kL; ++j) ps[j] = 0.0f;

    lds_u8* const d0 = (lds_u8*)s0;
    lds_u8* const d1 = (lds_u8*)s1;
    lds_u8* const d2 = (lds_u8*)s2;
    chunk_copy<P>(rs, d0, voff, 0, nch, 16u * U);
    chunk_copy<P>(rs, d1, voff, 1, nch, 16u * U);
    if (S > 2) chunk_copy<P>(rs, d2, voff, 2, nch, 16u * U);
    const uint8_t* r0 = s0 + lane * (16 * P);
    const uint8_t* r1 = s1 + lane * (16 * P);
    const uint8_t* r2 = s2 + lane * (16 * P);

    int ch = 0;
    for (; ch + S <= nfull; ch += S) {
        stage_step<U, S>(rs, d0, r0, voff, xw, ch, nch, ps);
        stage_step<U, S>(rs, d1, r1, voff, xw, ch + 1, nch, ps);
        if (S > 2) stage_step<U, S>(rs, d2, r2, voff, xw, ch + 2, nch, ps);
    }
    // Fewer than S full chunks and the tail remain, in stages 0, 1, 2 in order.
    __builtin_amdgcn_s_waitcnt(mg::kWaitVm0);
    const uint8_t* rr[3] = {r0, r1, r2};
#pragma unroll
    for (int st = 0; st < S; ++st) {
        const int c = ch + st;
        if (c < nfull)
            chunk_sum<U>(rr[st], xw + (int64_t)c * (4 * U), U, ps);
        else if (c == nfull && tail_units)
            chunk_sum<U>(rr[st], xw + (int64_t)c * (4 * U), tail_units, ps);
    }

    const float a01 = ps[0] + ps[1];
    const float a23 = ps[2] + ps[3];
    const float a45 = ps[4] + ps[5];
    const float a6 = ps[6] + 0.0f;
    const float b0 = a01 + a23;
    const float b1 = a45 + a6;
    const uint32_t bits = bf16_rne(b0 + b1);

    uint64_t best = 0;
    if (lane < nrows) {
        if (logits) logits[row0 + lane] = (uint16_t)bits;
        best = ((uint64_t)bf16_key(bits) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(row0 + lane));
    }
    if (part) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) best = umax64(best, __shfl_xor(best, o, 64));
        if (lane == 0) part[blockIdx.x] = best;
    }
}

__global__ void __launch_bounds__(1024) k_lmhead_argmax(const uint64_t* __restrict__ part, int64_t n,
                                                        int32_t* __restrict__ out) {
    __shared__ uint64_t red[16];
    uint64_t best = kSentinel;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) best = umax64(best, part[i]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) best = umax64(best, __shfl_xor(best, o, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x < 64) {
        best = threadIdx.x < (blockDim.x >> 6) ? red[threadIdx.x] : 0;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) best = umax64(best, __shfl_xor(best, o, 64));
        if (threadIdx.x == 0) out[0] = (int32_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu));
    }
}

}  // namespace lm

int64_t lm_head_workspace_bytes(int64_t V) { return (V + lm::kRows - 1) / lm::kRows * 8; }

hipError_t launch_lm_head(const void* w, int64_t V, int64_t K, const uint16_t* x, uint16_t* logits,
                          int32_t* argmax, void* ws, hipStream_t st) {
    const int64_t nwaves = (V + lm::kRows - 1) / lm::kRows;
    uint64_t* part = argmax ? static_cast<uint64_t*>(ws) : nullptr;
    hipLaunchKernelGGL((lm::k_lmhead<lm::kU, lm::kS>), dim3((unsigned)nwaves), dim3(64), 0, st, static_cast<const uint8_t*>(w), V, K, x,
                       logits, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !argmax) return e;
    hipLaunchKernelGGL(lm::k_lmhead_argmax, dim3(1), dim3(1024), 0, st, part, nwaves, argmax);
    return hipGetLastError();
}

}  // namespace aipu
