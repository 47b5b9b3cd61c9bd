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
// own row in k order.  The rows stream through LDS in chunks of 56 bf16 (112 B per row,
// a multiple of 7 so every chunk starts on partial sum 0): seven direct-to-LDS copies per
// chunk fill 64 rows x 112 B (row r at byte 112 r, 16-B unit u at 16 u), and each lane
// then reads its row back with seven 16-B LDS reads (112 B = 28 dwords: eight consecutive
// rows hit disjoint banks).  Two LDS stages per wave keep one chunk in flight while the
// previous one is summed; a workgroup is one wave, 14 KB of LDS, so the whole vocabulary
// of 154,880 rows (2,420 waves) is resident at once on 256 CUs.
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
constexpr int kUnits = 7;                  // 16-B units per row per chunk
constexpr int kChunk = kUnits * 8;         // 56 bf16 per row per chunk
constexpr int kRowBytes = kUnits * 16;     // 112
constexpr int kStageBytes = kRows * kRowBytes;   // 7168

// Order key of a bf16 pattern under bf16_gt: sign-magnitude, +0 == -0.
__device__ __forceinline__ uint32_t bf16_key(uint32_t b) {
    const uint32_t m = b & 0x7FFFu;
    return (b & 0x8000u) ? 0x8000u - m : 0x8000u + m;
}

// The starting candidate of the reference scan: -inf at index 0.
constexpr uint64_t kSentinel = ((uint64_t)(0x8000u - 0x7F80u) << 32) | 0xFFFFFFFFull;

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Seven partial sums of one lane over `nu` 16-B units of its row in LDS (nu = 7 except in
// the last chunk); xs points at the chunk's 56 activation values (wave-uniform).
template <bool kFull>
__device__ __forceinline__ void chunk_sum(const uint8_t* row, const uint32_t* __restrict__ xs, int nu,
                                          float (&ps)[kL]) {
    uint4 v[kUnits];
#pragma unroll
    for (int u = 0; u < kUnits; ++u)
        if (kFull || u < nu) v[u] = *reinterpret_cast<const uint4*>(row + 16 * u);
#pragma unroll
    for (int u = 0; u < kUnits; ++u) {
        if (!kFull && u >= nu) break;
        const uint32_t wd[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int e = 8 * u + 2 * h;          // element index within the chunk
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

// Issue the seven copies of chunk `ch` into one stage (all lanes read zeros without a
// memory access when ch is past the end: the offset lands outside the buffer).
typedef __attribute__((address_space(3))) uint8_t lds_u8;

__device__ __forceinline__ void chunk_copy(__amdgpu_buffer_rsrc_t rs, lds_u8* stage, const uint32_t (&voff)[kUnits],
                                           int ch, int nch) {
    const uint32_t soff = ch < nch ? (uint32_t)ch * kRowBytes : mg::kOOB;
#pragma unroll
    for (int c = 0; c < kUnits; ++c)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(stage + 1024 * c), 16,
                                                 voff[c], soff, 0, mg::kNT);
}

__global__ void __launch_bounds__(64) k_lmhead(const uint8_t* __restrict__ W, int64_t V, int64_t K,
                                               const uint16_t* __restrict__ x, uint16_t* __restrict__ logits,
                                               uint64_t* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) uint8_t s0[kStageBytes];
    __shared__ __attribute__((aligned(16))) uint8_t s1[kStageBytes];
    const int lane = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * kRows;
    const int64_t nrows = V - row0 < kRows ? V - row0 : kRows;
    const uint32_t rb = (uint32_t)(K * 2);                 // bytes per row
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(W + row0 * (int64_t)rb, (uint32_t)nrows * rb);

    // Copy c, lane l fills LDS unit p = 64c + l = 7r + u: row r, unit u of the chunk.
    uint32_t voff[kUnits];
#pragma unroll
    for (int c = 0; c < kUnits; ++c) {
        const int p = 64 * c + lane;
        voff[c] = (uint32_t)(p / kUnits) * rb + 16u * (uint32_t)(p % kUnits);
    }

    const int nfull = (int)(K / kChunk);
    const int tail_units = (int)((K % kChunk) / 8);
    const int nch = nfull + (tail_units ? 1 : 0);
    const uint32_t* xw = reinterpret_cast<const uint32_t*>(x);

    float ps[kL];
#pragma unroll
    for (int j = 0; j < kL; ++j) ps[j] = 0.0f;

    lds_u8* const d0 = (lds_u8*)s0;
    lds_u8* const d1 = (lds_u8*)s1;
    chunk_copy(rs, d0, voff, 0, nch);
    chunk_copy(rs, d1, voff, 1, nch);
    const uint8_t* r0 = s0 + lane * kRowBytes;
    const uint8_t* r1 = s1 + lane * kRowBytes;

    // Full chunks in pairs (stage 0, stage 1); copies for ch + 2 go out as soon as the
    // stage has been read into registers.
    int ch = 0;
    for (; ch + 1 < nfull; ch += 2) {
        __builtin_amdgcn_s_waitcnt(mg::kWaitVm0 | kUnits);   // vmcnt(7): stage 0 landed
        chunk_sum<true>(r0, xw + (int64_t)ch * (kChunk / 2), kUnits, ps);
        __builtin_amdgcn_s_waitcnt(mg::kWaitLgkm0);
        chunk_copy(rs, d0, voff, ch + 2, nch);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(mg::kWaitVm0 | kUnits);
        chunk_sum<true>(r1, xw + (int64_t)(ch + 1) * (kChunk / 2), kUnits, ps);
        __builtin_amdgcn_s_waitcnt(mg::kWaitLgkm0);
        chunk_copy(rs, d1, voff, ch + 3, nch);
        __builtin_amdgcn_sched_barrier(0);
    }
    // At most one full chunk (in stage 0) and the tail chunk remain.
    __builtin_amdgcn_s_waitcnt(mg::kWaitVm0);
    if (ch < nfull) {
        chunk_sum<true>(r0, xw + (int64_t)ch * (kChunk / 2), kUnits, ps);
        if (tail_units) chunk_sum<false>(r1, xw + (int64_t)(ch + 1) * (kChunk / 2), tail_units, ps);
    } else if (tail_units) {
        chunk_sum<false>(r0, xw + (int64_t)ch * (kChunk / 2), tail_units, ps);
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
    hipLaunchKernelGGL(lm::k_lmhead, dim3((unsigned)nwaves), dim3(64), 0, st, static_cast<const uint8_t*>(w), V, K, x,
                       logits, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !argmax) return e;
    hipLaunchKernelGGL(lm::k_lmhead_argmax, dim3(1), dim3(1024), 0, st, part, nwaves, argmax);
    return hipGetLastError();
}

}  // namespace aipu
