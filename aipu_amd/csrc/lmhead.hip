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
//
// For K <= 6720 (MODEL_DIM 6144) the launcher runs k_lmhead_rc below instead, whose lanes are
// (row, partial sum) pairs: 896-B row segments, 5.98 TB/s at 154,880 x 6,144 against 4.94 TB/s
// for the lane-per-row kernel, which stays for larger K.
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
    __builtin_amdgcn_s_waitcnt(mg::wait_vm((S - 1) * P));
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

// ------------------------------------------------------------- row x partial-sum lanes
// For K <= 7168: lane = (row r, partial sum j), 7 lanes per row, 9 rows per wave (lane 63
// duplicates row 8 and writes nothing), 4 waves per workgroup.  Each chunk is 448 bf16 of a
// row (64 products per partial sum), so every row segment a wave copies is 896 contiguous
// bytes -- twice the 448-B segments of the lane-per-row kernel, with a quarter of its LDS per
// row.  Lane (r, j) reads its products' weights with 2-B LDS reads at stride 14 B and its
// activations from a copy of x laid out by partial sum (xs[j][i] = x[7 i + j], staged once
// per workgroup), then the seven partial sums of a row meet through lane shuffles for the
// fixed add tree.  Elements past K are zeros in both the weight stage (the copies of the last
// chunk read nothing there) and xs, and adding +0 leaves a partial sum unchanged (a partial
// sum is never -0: it starts at +0 and x + (-x) rounds to +0).
constexpr int kRcRows = 9;
constexpr int kRcWaves = 4;
constexpr int kRcChunk = 448;                          // bf16 per row per chunk
constexpr int kRcUnits = kRcChunk * 2 / 16;            // 56 data units of 16 B
constexpr int kRcPitch = (kRcUnits + 1) * 16;          // 912 B: + one pad unit
// The last row needs no pad unit, so a stage is exactly 8 copies of 64 x 16 B: each copy
// writes a whole 1 KB (its lanes past the data read nothing and write zeros), so the stage
// must be a whole number of copies or the last copy would spill into the next wave's stage.
constexpr int kRcStage = kRcRows * kRcPitch - 16;      // 8192 B per wave and stage
constexpr int kRcCopies = kRcStage / 1024;             // 8
static_assert(kRcCopies * 1024 == kRcStage, "stage = whole copies");
constexpr int kRcMaxChunks = 15;                       // K <= 6720 (LDS for two workgroups per CU)

__host__ __device__ constexpr int rc_xs_pitch(int nch) { return nch * 128 + 16; }   // bytes per partial sum
__host__ __device__ constexpr int rc_xs_bytes(int nch) { return 7 * rc_xs_pitch(nch); }

__device__ __forceinline__ void rc_copy(__amdgpu_buffer_rsrc_t rs, lds_u8* stage, const uint32_t (&voff)[kRcCopies],
                                        const uint32_t (&unit)[kRcCopies], int ch, int nch, uint32_t lim) {
    const uint32_t soff = ch < nch ? (uint32_t)ch * (kRcChunk * 2) : mg::kOOB;
#pragma unroll
    for (int c = 0; c < kRcCopies; ++c) {
        const uint32_t v = unit[c] < lim ? voff[c] : mg::kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(stage + 1024 * c), 16,
                                                 v, soff, 0, mg::kNT);
    }
}

// 64 products of partial sum j of this lane's row: weights at wp + 14 i, activations xs[j][64 ch + i].
__device__ __forceinline__ float rc_chunk(const uint8_t* wp, const uint8_t* xp, float ps) {
#pragma unroll
    for (int i8 = 0; i8 < 8; ++i8) {
        const uint4 xv = *reinterpret_cast<const uint4*>(xp + 16 * i8);
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int i = 8 * i8 + q;
            const uint32_t wb = *reinterpret_cast<const uint16_t*>(wp + 14 * i);
            const float xf = __uint_as_float((q & 1) ? (xw[q >> 1] & 0xFFFF0000u) : (xw[q >> 1] << 16));
            ps = ps + xf * __uint_as_float(wb << 16);
        }
    }
    return ps;
}

__global__ void __launch_bounds__(64 * kRcWaves) k_lmhead_rc(const uint8_t* __restrict__ W, int64_t V, int64_t K,
                                                             const uint16_t* __restrict__ x,
                                                             uint16_t* __restrict__ logits,
                                                             uint64_t* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) uint8_t s0[kRcWaves * kRcStage];
    __shared__ __attribute__((aligned(16))) uint8_t s1[kRcWaves * kRcStage];
    __shared__ uint64_t wbest[kRcWaves];
    // a separate static object, so the compiler sees that reading it does not depend on the
    // weight copies still in flight into s0 / s1
    __shared__ __attribute__((aligned(16))) uint8_t xs[rc_xs_bytes(kRcMaxChunks)];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nch = (int)((K + kRcChunk - 1) / kRcChunk);
    const int ni = nch * 64;                     // products per partial sum, padded
    const int xpitch = rc_xs_pitch(nch);

    // 1. x by partial sum, zeros past K
    for (int idx = tid; idx < 7 * ni; idx += 64 * kRcWaves) {
        const int j = idx / ni, i = idx - j * ni;
        const int64_t k = 7 * (int64_t)i + j;
        *reinterpret_cast<uint16_t*>(xs + j * xpitch + 2 * i) = k < K ? x[k] : (uint16_t)0;
    }
    __syncthreads();

    // 2. this wave's rows
    const int64_t row0 = ((int64_t)blockIdx.x * kRcWaves + w) * kRcRows;
    const int64_t nrows = V - row0 < kRcRows ? (V - row0 > 0 ? V - row0 : 0) : kRcRows;
    const uint32_t rb = (uint32_t)(K * 2);
    const int r = lane / 7 < kRcRows ? lane / 7 : kRcRows - 1;
    const int j = lane - 7 * (lane / 7) < 7 && lane < 63 ? lane - 7 * (lane / 7) : 0;
    float ps = 0.0f;
    if (nrows > 0) {
        const __amdgpu_buffer_rsrc_t rs = buf_rsrc(W + row0 * (int64_t)rb, (uint32_t)nrows * rb);
        uint32_t voff[kRcCopies], unit[kRcCopies];
#pragma unroll
        for (int c = 0; c < kRcCopies; ++c) {
            const int p = 64 * c + lane;
            const int rr = p / (kRcUnits + 1), u = p - rr * (kRcUnits + 1);
            const bool ok = rr < kRcRows && u < kRcUnits;
            voff[c] = ok ? (uint32_t)rr * rb + 16u * (uint32_t)u : mg::kOOB;
            unit[c] = ok ? (uint32_t)u : 0xFFFFu;
        }
        const int nfull = (int)(K / kRcChunk);
        const uint32_t tail = (uint32_t)((K % kRcChunk) / 8);   // 16-B units of the last chunk
        lds_u8* const d0 = (lds_u8*)s0 + w * kRcStage;
        lds_u8* const d1 = (lds_u8*)s1 + w * kRcStage;
        rc_copy(rs, d0, voff, unit, 0, nch, 0 < nfull ? kRcUnits : tail);
        rc_copy(rs, d1, voff, unit, 1, nch, 1 < nfull ? kRcUnits : tail);
        const uint8_t* w0 = s0 + w * kRcStage + r * kRcPitch + 2 * j;
        const uint8_t* w1 = s1 + w * kRcStage + r * kRcPitch + 2 * j;
        const uint8_t* xj = xs + j * xpitch;
        int ch = 0;
        for (; ch + 1 < nch; ch += 2) {
            __builtin_amdgcn_s_waitcnt(mg::wait_vm(kRcCopies));
            ps = rc_chunk(w0, xj + ch * 128, ps);
            __builtin_amdgcn_s_waitcnt(mg::kWaitLgkm0);
            rc_copy(rs, d0, voff, unit, ch + 2, nch, ch + 2 < nfull ? kRcUnits : tail);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(mg::wait_vm(kRcCopies));
            ps = rc_chunk(w1, xj + (ch + 1) * 128, ps);
            __builtin_amdgcn_s_waitcnt(mg::kWaitLgkm0);
            rc_copy(rs, d1, voff, unit, ch + 3, nch, ch + 3 < nfull ? kRcUnits : tail);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(mg::kWaitVm0);
        if (ch < nch) ps = rc_chunk(w0, xj + ch * 128, ps);
    }

    // 3. the row's seven partial sums meet on every lane of the row; fixed tree; argmax
    float p[kL];
#pragma unroll
    for (int q = 0; q < kL; ++q) p[q] = __shfl(ps, 7 * r + q, 64);
    const float a01 = p[0] + p[1];
    const float a23 = p[2] + p[3];
    const float a45 = p[4] + p[5];
    const float a6 = p[6] + 0.0f;
    const uint32_t bits = bf16_rne((a01 + a23) + (a45 + a6));
    uint64_t best = 0;
    if (lane < 63 && j == 0 && r < nrows) {
        if (logits) logits[row0 + r] = (uint16_t)bits;
        best = ((uint64_t)bf16_key(bits) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)(row0 + r));
    }
    if (part) {
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) best = umax64(best, __shfl_xor(best, o, 64));
        if (lane == 0) wbest[w] = best;
        __syncthreads();
        if (tid == 0) {
            uint64_t b = wbest[0];
            for (int q = 1; q < kRcWaves; ++q) b = umax64(b, wbest[q]);
            part[blockIdx.x] = b;
        }
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

int64_t lm_head_workspace_bytes(int64_t V) {
    // one (key, -index) pair per workgroup of whichever kernel runs (the smaller of the two)
    const int64_t a = (V + lm::kRows - 1) / lm::kRows;
    const int64_t b = (V + lm::kRcRows * lm::kRcWaves - 1) / (lm::kRcRows * lm::kRcWaves);
    return (a > b ? a : b) * 8;
}

hipError_t launch_lm_head(const void* w, int64_t V, int64_t K, const uint16_t* x, uint16_t* logits,
                          int32_t* argmax, void* ws, hipStream_t st) {
    uint64_t* part = argmax ? static_cast<uint64_t*>(ws) : nullptr;
    int64_t nparts;
    if (K <= (int64_t)lm::kRcChunk * lm::kRcMaxChunks) {
        nparts = (V + lm::kRcRows * lm::kRcWaves - 1) / (lm::kRcRows * lm::kRcWaves);
        hipLaunchKernelGGL(lm::k_lmhead_rc, dim3((unsigned)nparts), dim3(64 * lm::kRcWaves), 0, st,
                           static_cast<const uint8_t*>(w), V, K, x, logits, part);
    } else {
        nparts = (V + lm::kRows - 1) / lm::kRows;
        hipLaunchKernelGGL((lm::k_lmhead<lm::kU, lm::kS>), dim3((unsigned)nparts), dim3(64), 0, st,
                           static_cast<const uint8_t*>(w), V, K, x, logits, part);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !argmax) return e;
    hipLaunchKernelGGL(lm::k_lmhead_argmax, dim3(1), dim3(1024), 0, st, part, nparts, argmax);
    return hipGetLastError();
}

}  // namespace aipu
