// Reference-order GEMV: bit-identical to the reference's golden for every ggml type.
//
// Contract (tools/q4k_ref.py:67-92, RTL order src/glm_matmul_q4k.v:261-270): for each
// output (m, n) the weight row is dequantised exactly and
//     acc = f32(acc + f32(x[m][k] * w[n][k]))     for k = 0 .. K-1, in order,
// then y = bf16_RNE(acc).  One lane owns one output row and walks K sequentially.  Q4_K with
// K <= 32768 runs k_gemv_ref_q4k (row blocks in registers, activations staged once as fp32),
// Q8_0 / F16 / BF16 with K a multiple of 64 k_gemv_ref_reg and Q6_K with K a multiple of 512
// k_gemv_ref_q6k (the same for their blocks), all with aligned pointers; larger K, other K and
// unaligned pointers run k_gemv_ref, whose 64 rows per workgroup are staged 256
// weights at a time through LDS so the global reads stay coalesced, with a last stage of fewer
// weights for K that is a multiple of the type's block but not of 256 (Q8_0: 32; F16 / BF16:
// any K).  The library is compiled with -ffp-contract=off, so the multiply and the add below
// are two separately rounded ops.
#include "common.hpp"
#include "launch.hpp"

namespace aipu {

namespace {

constexpr int kRows = 64;      // rows per workgroup (one wave)
constexpr int kMC = 8;         // activation rows per pass (blockIdx.y walks the rest)
constexpr int kStageW = 256;   // weights per stage

template <int TYPE>
struct Stage {
    static constexpr int bytes = (int)row_bytes(TYPE, kStageW);    // per row per stage
    static constexpr int u16 = bytes / 2;
    static constexpr int stride = u16 + ((u16 & 1) ? 0 : 1);        // odd stride in u16 words
};

// Dequantise weight k (0..255) of the row's current stage, reading the staged bytes.
// Q4_K: tools/q4k_ref.py:45-60.  Computed per 32-weight sub-block by the caller.
template <int TYPE>
__device__ __forceinline__ void stage_mac(const uint8_t* rb, const float (*xs)[kStageW], int mcnt, float* acc,
                                          int kn) {
    if constexpr (TYPE == T_Q4_K) {
        const uint16_t* h = (const uint16_t*)rb;
        const float d = f16_to_f32(h[0]);
        const float dm = f16_to_f32(h[1]);
        uint32_t s[3];
#pragma unroll
        for (int i = 0; i < 3; ++i)
            s[i] = (uint32_t)rb[4 + 4 * i] | ((uint32_t)rb[5 + 4 * i] << 8) | ((uint32_t)rb[6 + 4 * i] << 16) |
                   ((uint32_t)rb[7 + 4 * i] << 24);
        const uint8_t* qs = rb + 16;
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, m;
            q4k_scale_min(j, s[0], s[1], s[2], sc, m);
            const float D = d * (float)sc;
            const float Mn = dm * (float)m;
            const int g = j >> 1, hi = j & 1;
            for (int l = 0; l < 32; ++l) {
                const uint32_t q = hi ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 0xFu);
                const float w = q4k_weight_exact(D, Mn, q);
                const int k = 32 * j + l;
                for (int mm = 0; mm < kMC; ++mm) {
                    if (mm < mcnt) {
                        const float p = xs[mm][k] * w;
                        acc[mm] = acc[mm] + p;
                    }
                }
            }
        }
    } else if constexpr (TYPE == T_Q6_K) {
        // ql[128] qh[64] int8 sc[16] fp16 d  (tools/q4k_ref.py:105-124)
        const float d = f16_to_f32((uint32_t)rb[208] | ((uint32_t)rb[209] << 8));
        for (int k = 0; k < 256; ++k) {
            const int h = k >> 7, t = (k >> 5) & 3, l = k & 31;
            const uint32_t qlb = rb[64 * h + l + 32 * (t & 1)];
            const uint32_t nib = t < 2 ? (qlb & 0xFu) : (qlb >> 4);
            const uint32_t code = nib | ((((uint32_t)rb[128 + 32 * h + l]) >> (2 * t)) & 3u) << 4;
            const float ds = d * (float)(int8_t)rb[192 + (k >> 4)];
            const float w = ds * (float)((int)code - 32);
            for (int mm = 0; mm < kMC; ++mm) {
                if (mm < mcnt) {
                    const float p = xs[mm][k] * w;
                    acc[mm] = acc[mm] + p;
                }
            }
        }
    } else if constexpr (TYPE == T_Q8_0) {
        // up to 8 blocks of fp16 d | int8 qs[32]  (tools/q4k_ref.py:126-129)
        for (int b = 0; b < kn / 32; ++b) {
            const uint8_t* p8 = rb + 34 * b;
            const float d = f16_to_f32((uint32_t)p8[0] | ((uint32_t)p8[1] << 8));
            for (int i = 0; i < 32; ++i) {
                const float w = d * (float)(int8_t)p8[2 + i];
                const int k = 32 * b + i;
                for (int mm = 0; mm < kMC; ++mm) {
                    if (mm < mcnt) {
                        const float p = xs[mm][k] * w;
                        acc[mm] = acc[mm] + p;
                    }
                }
            }
        }
    } else {  // F16 / BF16 passthrough
        const uint16_t* h = (const uint16_t*)rb;
        for (int k = 0; k < kn; ++k) {
            const float w = TYPE == T_F16 ? f16_to_f32(h[k]) : bf16_to_f32(h[k]);
            for (int mm = 0; mm < kMC; ++mm) {
                if (mm < mcnt) {
                    const float p = xs[mm][k] * w;
                    acc[mm] = acc[mm] + p;
                }
            }
        }
    }
}

// Slot gathering (MoE): blockIdx.z = slot z reads weight matrix sel[z] of the `_exps`
// stack at W + sel[z]*wstride when z < topk, else W_alt (the shared expert); activations
// and outputs are offset by z*x_zstride / z*y_zstride.  Plain GEMV: sel == nullptr, z = 0.
struct RefGather {
    const int32_t* sel;
    int topk;
    int64_t E;
    int64_t wstride;
    const uint8_t* W_alt;
    int64_t x_zstride;
    int64_t y_zstride;
};

template <int TYPE>
__global__ __launch_bounds__(kRows) void k_gemv_ref(const uint8_t* __restrict__ W, int64_t N, int64_t K,
                                                    const uint16_t* __restrict__ X, int64_t M,
                                                    uint16_t* __restrict__ Y, float* __restrict__ Yf,
                                                    RefGather ga) {
    using S = Stage<TYPE>;
    if (ga.sel) {
        const int z = blockIdx.z;
        if (z < ga.topk) {
            int e = ga.sel[z];
            e = e < 0 ? 0 : (e >= ga.E ? (int)ga.E - 1 : e);
            W += (int64_t)e * ga.wstride;
        } else {
            W = ga.W_alt;
        }
        X += (int64_t)z * ga.x_zstride;
        Y += (int64_t)z * ga.y_zstride;
        if (Yf) Yf += (int64_t)z * ga.y_zstride;
    }
    __shared__ uint16_t rows[kRows * S::stride];
    __shared__ float xs[kMC][kStageW];
    const int lane = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * kRows;
    const int64_t m0 = (int64_t)blockIdx.y * kMC;
    const int mcnt = (int)((M - m0) < kMC ? (M - m0) : kMC);
    const int64_t rb = row_bytes(TYPE, K);
    const int nfull = (int)(K / kStageW);
    const int ktail = (int)(K - (int64_t)nfull * kStageW);   // a multiple of the type's block
    float acc[kMC];
#pragma unroll
    for (int i = 0; i < kMC; ++i) acc[i] = 0.0f;

    for (int st = 0; st < nfull + (ktail ? 1 : 0); ++st) {
        const int kn = st < nfull ? kStageW : ktail;
        __syncthreads();
        if (kn == kStageW) {
            for (int idx = lane; idx < kRows * S::u16; idx += kRows) {
                const int r = idx / S::u16, c = idx - r * S::u16;
                const int64_t n = row0 + r;
                uint16_t v = 0;
                if (n < N) v = *(const uint16_t*)(W + n * rb + (int64_t)st * S::bytes + 2 * c);
                rows[r * S::stride + c] = v;
            }
        } else {
            const int u16 = (int)(row_bytes(TYPE, kn) / 2);   // Q8_0: 17 words per block; F16 / BF16: kn
            for (int idx = lane; idx < kRows * u16; idx += kRows) {
                const int r = idx / u16, c = idx - r * u16;
                const int64_t n = row0 + r;
                uint16_t v = 0;
                if (n < N) v = *(const uint16_t*)(W + n * rb + (int64_t)st * S::bytes + 2 * c);
                rows[r * S::stride + c] = v;
            }
        }
        for (int idx = lane; idx < kMC * kStageW; idx += kRows) {
            const int mm = idx / kStageW, k = idx - mm * kStageW;
            xs[mm][k] = mm < mcnt && k < kn ? bf16_to_f32(X[(m0 + mm) * K + (int64_t)st * kStageW + k]) : 0.0f;
        }
        __syncthreads();
        if (row0 + lane < N) stage_mac<TYPE>((const uint8_t*)(rows + lane * S::stride), xs, mcnt, acc, kn);
    }
    const int64_t n = row0 + lane;
    if (n < N) {
        for (int mm = 0; mm < mcnt; ++mm) {
            Y[(m0 + mm) * N + n] = (uint16_t)bf16_rne(acc[mm]);
            if (Yf) Yf[(m0 + mm) * N + n] = acc[mm];
        }
    }
}

// Q4_K in reference order with the weights in registers: the same operations in the same order
// as k_gemv_ref<T_Q4_K> (so the same bits), arranged for the VALU.  Lane = output row; each
// lane loads its row's 144-B super-block with nine 16-B loads, one block ahead of its use, and
// the MC activation rows of the pass sit in LDS as fp32 (staged once, MC * K * 4 bytes), read
// four at a time by every lane of the wave at one address.  Per weight: the nibble, its fp32
// value (one byte conversion), w = D q - Mn, and for every activation row acc += x w.
constexpr int kRefQ4LdsBytes = 128 * 1024;   // staged activations, at most

// Byte B of v as fp32 in one instruction (plain C selects a bit-field extract, then the
// conversion of byte 0).  VALU only, no hazard beyond what the hardware interlocks.
template <int B>
__device__ __forceinline__ float cvt_ubyte(uint32_t v) {
    float r;
    if constexpr (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if constexpr (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

template <int MC>
__global__ __launch_bounds__(kRows) void k_gemv_ref_q4k(const uint8_t* __restrict__ W, int64_t N, int64_t K,
                                                        const uint16_t* __restrict__ X, int64_t M,
                                                        uint16_t* __restrict__ Y, float* __restrict__ Yf,
                                                        RefGather ga) {
    if (ga.sel) {
        const int z = blockIdx.z;
        if (z < ga.topk) {
            int e = ga.sel[z];
            e = e < 0 ? 0 : (e >= ga.E ? (int)ga.E - 1 : e);
            W += (int64_t)e * ga.wstride;
        } else {
            W = ga.W_alt;
        }
        X += (int64_t)z * ga.x_zstride;
        Y += (int64_t)z * ga.y_zstride;
        if (Yf) Yf += (int64_t)z * ga.y_zstride;
    }
    extern __shared__ __align__(16) float s_x[];   // [MC][K]
    const int lane = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * kRows;
    const int64_t m0 = (int64_t)blockIdx.y * MC;
    const int mcnt = (int)((M - m0) < MC ? (M - m0) : MC);
    const int nsb = (int)(K / QK_K);
    const uint32_t rb = (uint32_t)nsb * 144u;
    const int nrows = (int)((N - row0) < kRows ? (N - row0) : kRows);
    // this lane's row (rows past N read zeros), one block ahead
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W + row0 * (int64_t)rb, (uint32_t)nrows * rb);
    const uint32_t wrow = (uint32_t)lane * rb;
    uint4 nxt[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) nxt[i] = buf_load16(wr, wrow + 16u * (uint32_t)i);
    // the pass's activation rows as fp32 (rows past M as zeros): chunks of 8 elements, eight
    // chunks' loads in flight before their stores
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X + m0 * K, (uint32_t)mcnt * (uint32_t)K * 2u);
    const int nch = MC * (int)(K / 8);
    for (int c0 = 0; c0 < nch; c0 += 8 * kRows) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kRows + lane;
            v[u] = buf_load16(xr, c < nch ? 16u * (uint32_t)c : 0xF0000000u);   // chunk c: row c / (K / 8)
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kRows + lane;
            if (c < nch) {
                float4* d = (float4*)(s_x + 8 * (int64_t)c);
                d[0] = make_float4(bf16_to_f32(v[u].x & 0xFFFFu), bf16_to_f32(v[u].x >> 16),
                                   bf16_to_f32(v[u].y & 0xFFFFu), bf16_to_f32(v[u].y >> 16));
                d[1] = make_float4(bf16_to_f32(v[u].z & 0xFFFFu), bf16_to_f32(v[u].z >> 16),
                                   bf16_to_f32(v[u].w & 0xFFFFu), bf16_to_f32(v[u].w >> 16));
            }
        }
    }
    __syncthreads();
    float acc[MC];
#pragma unroll
    for (int i = 0; i < MC; ++i) acc[i] = 0.0f;
    for (int b = 0; b < nsb; ++b) {
        uint4 R[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) R[i] = nxt[i];
        if (b + 1 < nsb) {
#pragma unroll
            for (int i = 0; i < 9; ++i) nxt[i] = buf_load16(wr, wrow + 144u * (uint32_t)(b + 1) + 16u * (uint32_t)i);
        }
        // tools/q4k_ref.py:45-60: d, dmin, the packed scales, then the 128 bytes of nibbles
        const float d = f16_to_f32(R[0].x & 0xFFFFu);
        const float dm = f16_to_f32(R[0].x >> 16);
        const uint32_t s0 = R[0].y, s1 = R[0].z, s2 = R[0].w;
        const uint32_t qd[32] = {R[1].x, R[1].y, R[1].z, R[1].w, R[2].x, R[2].y, R[2].z, R[2].w,
                                 R[3].x, R[3].y, R[3].z, R[3].w, R[4].x, R[4].y, R[4].z, R[4].w,
                                 R[5].x, R[5].y, R[5].z, R[5].w, R[6].x, R[6].y, R[6].z, R[6].w,
                                 R[7].x, R[7].y, R[7].z, R[7].w, R[8].x, R[8].y, R[8].z, R[8].w};
        const float* xb = s_x + (int64_t)b * QK_K;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sc, mn;
            q4k_scale_min(j, s0, s1, s2, sc, mn);
            const float D = d * (float)sc;
            const float Mn = dm * (float)mn;
            const int g = j >> 1, hi = j & 1;
#pragma unroll
            for (int c = 0; c < 8; ++c) {   // bytes 4c .. 4c + 3 of the 32 of sub-block pair g
                const uint32_t v = (hi ? qd[8 * g + c] >> 4 : qd[8 * g + c]) & 0x0F0F0F0Fu;
                const float q[4] = {cvt_ubyte<0>(v), cvt_ubyte<1>(v), cvt_ubyte<2>(v), cvt_ubyte<3>(v)};
                const int k = 32 * j + 4 * c;
                float4 xv[MC];
#pragma unroll
                for (int mm = 0; mm < MC; ++mm) xv[mm] = *(const float4*)(xb + (int64_t)mm * K + k);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float wq = D * q[e];   // q4k_weight_exact: D * q, then - Mn
                    const float we = wq - Mn;
#pragma unroll
                    for (int mm = 0; mm < MC; ++mm) {
                        const float xe = e == 0 ? xv[mm].x : e == 1 ? xv[mm].y : e == 2 ? xv[mm].z : xv[mm].w;
                        const float p = xe * we;
                        acc[mm] = acc[mm] + p;
                    }
                }
            }
        }
    }
    const int64_t n = row0 + lane;
    if (n < N) {
        for (int mm = 0; mm < mcnt; ++mm) {
            Y[(m0 + mm) * N + n] = (uint16_t)bf16_rne(acc[mm]);
            if (Yf) Yf[(m0 + mm) * N + n] = acc[mm];
        }
    }
}

// Q8_0, F16 and BF16 in reference order with the weights in registers, as k_gemv_ref_q4k does
// for Q4_K: the dequantisation of k_gemv_ref's stage_mac (so the same bits).  A unit is 64
// weights: two Q8_0 blocks (68 B, 17 dwords: needs K % 64 == 0 so every unit starts 4-B
// aligned) or 128 B of F16 / BF16 (needs K % 64 == 0 so rows start 16-B aligned).
template <int TYPE>
struct RegUnit {
    static constexpr int kDw = TYPE == T_Q8_0 ? 17 : 32;   // dwords per unit
    static constexpr int kBytes = 4 * kDw;
};

template <int TYPE, int MC>
__global__ __launch_bounds__(kRows) void k_gemv_ref_reg(const uint8_t* __restrict__ W, int64_t N, int64_t K,
                                                        const uint16_t* __restrict__ X, int64_t M,
                                                        uint16_t* __restrict__ Y, float* __restrict__ Yf,
                                                        RefGather ga) {
    typedef RegUnit<TYPE> U;
    if (ga.sel) {
        const int z = blockIdx.z;
        if (z < ga.topk) {
            int e = ga.sel[z];
            e = e < 0 ? 0 : (e >= ga.E ? (int)ga.E - 1 : e);
            W += (int64_t)e * ga.wstride;
        } else {
            W = ga.W_alt;
        }
        X += (int64_t)z * ga.x_zstride;
        Y += (int64_t)z * ga.y_zstride;
        if (Yf) Yf += (int64_t)z * ga.y_zstride;
    }
    extern __shared__ __align__(16) float s_x[];   // [MC][K]
    const int lane = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * kRows;
    const int64_t m0 = (int64_t)blockIdx.y * MC;
    const int mcnt = (int)((M - m0) < MC ? (M - m0) : MC);
    const int nu = (int)(K / 64);
    const uint32_t rb = (uint32_t)nu * (uint32_t)U::kBytes;
    const int nrows = (int)((N - row0) < kRows ? (N - row0) : kRows);
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W + row0 * (int64_t)rb, (uint32_t)nrows * rb);
    const uint32_t wrow = (uint32_t)lane * rb;
    uint32_t nxt[U::kDw];
    auto load_unit = [&](int u) {
        const uint32_t o = wrow + (uint32_t)U::kBytes * (uint32_t)u;
        if constexpr (TYPE == T_Q8_0) {
#pragma unroll
            for (int i = 0; i < U::kDw; ++i) nxt[i] = buf_load4(wr, o + 4u * (uint32_t)i);
        } else {
#pragma unroll
            for (int i = 0; i < U::kDw / 4; ++i) {
                const uint4 v = buf_load16(wr, o + 16u * (uint32_t)i);
                nxt[4 * i] = v.x;
                nxt[4 * i + 1] = v.y;
                nxt[4 * i + 2] = v.z;
                nxt[4 * i + 3] = v.w;
            }
        }
    };
    load_unit(0);
    // the pass's activation rows as fp32 (rows past M as zeros), eight loads in flight per lane
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X + m0 * K, (uint32_t)mcnt * (uint32_t)K * 2u);
    const int nch = MC * (int)(K / 8);
    for (int c0 = 0; c0 < nch; c0 += 8 * kRows) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kRows + lane;
            v[u] = buf_load16(xr, c < nch ? 16u * (uint32_t)c : 0xF0000000u);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kRows + lane;
            if (c < nch) {
                float4* d = (float4*)(s_x + 8 * (int64_t)c);
                d[0] = make_float4(bf16_to_f32(v[u].x & 0xFFFFu), bf16_to_f32(v[u].x >> 16),
                                   bf16_to_f32(v[u].y & 0xFFFFu), bf16_to_f32(v[u].y >> 16));
                d[1] = make_float4(bf16_to_f32(v[u].z & 0xFFFFu), bf16_to_f32(v[u].z >> 16),
                                   bf16_to_f32(v[u].w & 0xFFFFu), bf16_to_f32(v[u].w >> 16));
            }
        }
    }
    __syncthreads();
    float acc[MC];
#pragma unroll
    for (int i = 0; i < MC; ++i) acc[i] = 0.0f;
    for (int u = 0; u < nu; ++u) {
        uint32_t R[U::kDw];
#pragma unroll
        for (int i = 0; i < U::kDw; ++i) R[i] = nxt[i];
        if (u + 1 < nu) load_unit(u + 1);
        const float* xb = s_x + (int64_t)u * 64;
#pragma unroll
        for (int c = 0; c < 16; ++c) {   // weights 4c .. 4c + 3 of the unit
            float w[4];
            if constexpr (TYPE == T_Q8_0) {
                // block c / 8: fp16 d at bytes 34 (c / 8), codes at bytes 34 (c / 8) + 2 + ..
                const int blk = c >> 3, i0 = 4 * (c & 7);
                const float d = f16_to_f32(blk == 0 ? (R[0] & 0xFFFFu) : (R[8] >> 16));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int byte = 34 * blk + 2 + i0 + e;   // byte of the unit
                    const uint32_t q = (R[byte >> 2] >> (8 * (byte & 3))) & 0xFFu;
                    w[e] = d * (float)(int8_t)q;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t h = (R[2 * c + (e >> 1)] >> (16 * (e & 1))) & 0xFFFFu;
                    w[e] = TYPE == T_F16 ? f16_to_f32(h) : bf16_to_f32(h);
                }
            }
            float4 xv[MC];
#pragma unroll
            for (int mm = 0; mm < MC; ++mm) xv[mm] = *(const float4*)(xb + (int64_t)mm * K + 4 * c);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
#pragma unroll
                for (int mm = 0; mm < MC; ++mm) {
                    const float xe = e == 0 ? xv[mm].x : e == 1 ? xv[mm].y : e == 2 ? xv[mm].z : xv[mm].w;
                    const float p = xe * w[e];
                    acc[mm] = acc[mm] + p;
                }
            }
        }
    }
    const int64_t n = row0 + lane;
    if (n < N) {
        for (int mm = 0; mm < mcnt; ++mm) {
            Y[(m0 + mm) * N + n] = (uint16_t)bf16_rne(acc[mm]);
            if (Yf) Yf[(m0 + mm) * N + n] = acc[mm];
        }
    }
}

// Q6_K in reference order with the weights in registers: stage_mac's Q6_K dequantisation (so
// the same bits).  A 210-B block starts 4-B aligned when its index is even and 2 B past a dword
// when it is odd (K a multiple of 512, rows 4-B aligned); each lane loads the 53 dwords that
// span its block, one block ahead, and realigns the dwords it uses by `par` (0 or 2) bytes.
// Four weights at a time: code = nibble | 2-bit high part << 4 for four bytes in one dword,
// then per weight (float)(code - 32) (as cvt(code) - 32, exact) times d * sc.
__device__ __forceinline__ uint32_t q6_dword(const uint32_t (&R)[53], int o, uint32_t par) {   // bytes o .. o + 3, o % 4 == 0, o <= 204
    return __builtin_amdgcn_alignbyte(R[(o >> 2) + 1], R[o >> 2], par);
}

template <int MC>
__device__ __forceinline__ void q6_block_ref(const uint32_t (&R)[53], uint32_t par, const float* xb, int64_t K,
                                             float (&acc)[MC]) {
    const float d = f16_to_f32(par ? R[52] >> 16 : R[52] & 0xFFFFu);   // d: block bytes 208..209, the span's last dword
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            __builtin_amdgcn_sched_barrier(0);   // one run of 32 weights at a time (registers)
#pragma unroll
            for (int c = 0; c < 8; ++c) {   // weights 128h + 32t + 4c .. + 3
                const uint32_t ql = q6_dword(R, 64 * h + 32 * (t & 1) + 4 * c, par);
                const uint32_t qh = q6_dword(R, 128 + 32 * h + 4 * c, par);
                const uint32_t code = ((t < 2 ? ql : ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (2 * t)) & 0x03030303u) << 4);
                const int si = 8 * h + 2 * t + (c >> 2);   // scale index k >> 4
                const uint32_t sw = q6_dword(R, 192 + (si & ~3), par);
                const float ds = d * (float)(int8_t)(uint8_t)(sw >> (8 * (si & 3)));
                const float q[4] = {cvt_ubyte<0>(code), cvt_ubyte<1>(code), cvt_ubyte<2>(code), cvt_ubyte<3>(code)};
                const int k = 128 * h + 32 * t + 4 * c;
                float4 xv[MC];
#pragma unroll
                for (int mm = 0; mm < MC; ++mm) xv[mm] = *(const float4*)(xb + (int64_t)mm * K + k);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float w = ds * (q[e] - 32.0f);
#pragma unroll
                    for (int mm = 0; mm < MC; ++mm) {
                        const float xe = e == 0 ? xv[mm].x : e == 1 ? xv[mm].y : e == 2 ? xv[mm].z : xv[mm].w;
                        const float p = xe * w;
                        acc[mm] = acc[mm] + p;
                    }
                }
            }
        }
}

template <int MC>
__global__ __launch_bounds__(kRows) void k_gemv_ref_q6k(const uint8_t* __restrict__ W, int64_t N, int64_t K,
                                                        const uint16_t* __restrict__ X, int64_t M,
                                                        uint16_t* __restrict__ Y, float* __restrict__ Yf,
                                                        RefGather ga) {
    if (ga.sel) {
        const int z = blockIdx.z;
        if (z < ga.topk) {
            int e = ga.sel[z];
            e = e < 0 ? 0 : (e >= ga.E ? (int)ga.E - 1 : e);
            W += (int64_t)e * ga.wstride;
        } else {
            W = ga.W_alt;
        }
        X += (int64_t)z * ga.x_zstride;
        Y += (int64_t)z * ga.y_zstride;
        if (Yf) Yf += (int64_t)z * ga.y_zstride;
    }
    extern __shared__ __align__(16) float s_x[];   // [MC][K]
    const int lane = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * kRows;
    const int64_t m0 = (int64_t)blockIdx.y * MC;
    const int mcnt = (int)((M - m0) < MC ? (M - m0) : MC);
    const int nsb = (int)(K / QK_K);
    const uint32_t rb = (uint32_t)nsb * 210u;
    const int nrows = (int)((N - row0) < kRows ? (N - row0) : kRows);
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W + row0 * (int64_t)rb, (uint32_t)nrows * rb);
    const uint32_t wrow = (uint32_t)lane * rb;
    uint32_t nxt[53];
    auto load_block = [&](int b) {   // the dwords spanning block b (the last one may read past the row: zeros or junk)
        const uint32_t o = wrow + ((210u * (uint32_t)b) & ~3u);
#pragma unroll
        for (int i = 0; i < 53; ++i) nxt[i] = buf_load4(wr, o + 4u * (uint32_t)i);
    };
    load_block(0);
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X + m0 * K, (uint32_t)mcnt * (uint32_t)K * 2u);
    const int nch = MC * (int)(K / 8);
    for (int c0 = 0; c0 < nch; c0 += 8 * kRows) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kRows + lane;
            v[u] = buf_load16(xr, c < nch ? 16u * (uint32_t)c : 0xF0000000u);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * kRows + lane;
            if (c < nch) {
                float4* d = (float4*)(s_x + 8 * (int64_t)c);
                d[0] = make_float4(bf16_to_f32(v[u].x & 0xFFFFu), bf16_to_f32(v[u].x >> 16),
                                   bf16_to_f32(v[u].y & 0xFFFFu), bf16_to_f32(v[u].y >> 16));
                d[1] = make_float4(bf16_to_f32(v[u].z & 0xFFFFu), bf16_to_f32(v[u].z >> 16),
                                   bf16_to_f32(v[u].w & 0xFFFFu), bf16_to_f32(v[u].w >> 16));
            }
        }
    }
    __syncthreads();
    float acc[MC];
#pragma unroll
    for (int i = 0; i < MC; ++i) acc[i] = 0.0f;
    for (int b = 0; b < nsb; ++b) {
        uint32_t R[53];
#pragma unroll
        for (int i = 0; i < 53; ++i) R[i] = nxt[i];
        if (b + 1 < nsb) load_block(b + 1);
        q6_block_ref<MC>(R, (210u * (uint32_t)b) & 3u, s_x + (int64_t)b * QK_K, K, acc);
    }
    const int64_t n = row0 + lane;
    if (n < N) {
        for (int mm = 0; mm < mcnt; ++mm) {
            Y[(m0 + mm) * N + n] = (uint16_t)bf16_rne(acc[mm]);
            if (Yf) Yf[(m0 + mm) * N + n] = acc[mm];
        }
    }
}

// Reference order on already-dequantised fp32 weights (matmul_q4k_col on a wdeq column).
__global__ __launch_bounds__(kRows) void k_gemv_ref_f32(const float* __restrict__ W, int64_t N, int64_t K,
                                                        const float* __restrict__ X, int64_t M,
                                                        uint16_t* __restrict__ Y, float* __restrict__ Yf) {
    __shared__ float xs[kMC][kStageW];
    const int lane = threadIdx.x;
    const int64_t n = (int64_t)blockIdx.x * kRows + lane;
    const int64_t m0 = (int64_t)blockIdx.y * kMC;
    const int mcnt = (int)((M - m0) < kMC ? (M - m0) : kMC);
    float acc[kMC];
#pragma unroll
    for (int i = 0; i < kMC; ++i) acc[i] = 0.0f;
    for (int64_t k0 = 0; k0 < K; k0 += kStageW) {
        const int kn = (int)((K - k0) < kStageW ? (K - k0) : kStageW);
        __syncthreads();
        for (int idx = lane; idx < kMC * kStageW; idx += kRows) {
            const int mm = idx / kStageW, k = idx - mm * kStageW;
            xs[mm][k] = (mm < mcnt && k < kn) ? X[(m0 + mm) * K + k0 + k] : 0.0f;
        }
        __syncthreads();
        if (n < N) {
            for (int k = 0; k < kn; ++k) {
                const float w = W[n * K + k0 + k];
                for (int mm = 0; mm < kMC; ++mm) {
                    if (mm < mcnt) {
                        const float p = xs[mm][k] * w;
                        acc[mm] = acc[mm] + p;
                    }
                }
            }
        }
    }
    if (n < N) {
        for (int mm = 0; mm < mcnt; ++mm) {
            Y[(m0 + mm) * N + n] = (uint16_t)bf16_rne(acc[mm]);
            if (Yf) Yf[(m0 + mm) * N + n] = acc[mm];
        }
    }
}

}  // namespace

hipError_t launch_gemv_ref_gather(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                                  uint16_t* y, float* y_f32, int nslots, const int32_t* sel, int topk, int64_t E,
                                  int64_t wstride, const void* w_alt, int64_t x_zstride, int64_t y_zstride,
                                  hipStream_t st) {
    const uint8_t* W = (const uint8_t*)w;
    const RefGather ga{sel, topk, E, wstride, (const uint8_t*)w_alt, x_zstride, y_zstride};
    // the register kernels load 16 B of activations and whole dwords / 16 B of weights at a time:
    // the pointers they start from must be aligned for that (the ABI asks less in this mode)
    auto al = [](const void* p, uintptr_t a) { return p == nullptr || ((uintptr_t)p & (a - 1)) == 0; };
    const uintptr_t wa = (type == T_Q8_0 || type == T_Q6_K) ? 4 : 16;
    const bool reg_ok = al(x, 16) && al(w, wa) && al(w_alt, wa) && (x_zstride * 2) % 16 == 0 && wstride % (int64_t)wa == 0;
    if (reg_ok && type == T_Q4_K && K % QK_K == 0 && K * 4 <= kRefQ4LdsBytes) {
        // the register kernel: MC activation rows per pass, as many as the staged rows allow
        int mc = 8;
        while (mc > 1 && (mc / 2 >= M || (int64_t)mc * K * 4 > kRefQ4LdsBytes)) mc /= 2;
        const dim3 g4((unsigned)((N + kRows - 1) / kRows), (unsigned)((M + mc - 1) / mc), (unsigned)nslots);
        const size_t lds = (size_t)mc * (size_t)K * 4;
        switch (mc) {
            case 8: hipLaunchKernelGGL(k_gemv_ref_q4k<8>, g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break;
            case 4: hipLaunchKernelGGL(k_gemv_ref_q4k<4>, g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break;
            case 2: hipLaunchKernelGGL(k_gemv_ref_q4k<2>, g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break;
            default: hipLaunchKernelGGL(k_gemv_ref_q4k<1>, g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break;
        }
        return hipGetLastError();
    }
    if (reg_ok && type == T_Q6_K && K % 512 == 0 && K * 4 <= kRefQ4LdsBytes) {
        int mc = 8;
        while (mc > 1 && (mc / 2 >= M || (int64_t)mc * K * 4 > kRefQ4LdsBytes)) mc /= 2;
        const dim3 g4((unsigned)((N + kRows - 1) / kRows), (unsigned)((M + mc - 1) / mc), (unsigned)nslots);
        const size_t lds = (size_t)mc * (size_t)K * 4;
        switch (mc) {
            case 8: hipLaunchKernelGGL(k_gemv_ref_q6k<8>, g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break;
            case 4: hipLaunchKernelGGL(k_gemv_ref_q6k<4>, g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break;
            case 2: hipLaunchKernelGGL(k_gemv_ref_q6k<2>, g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break;
            default: hipLaunchKernelGGL(k_gemv_ref_q6k<1>, g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break;
        }
        return hipGetLastError();
    }
    if (reg_ok && (type == T_Q8_0 || type == T_F16 || type == T_BF16) && K % 64 == 0 && K * 4 <= kRefQ4LdsBytes) {
        int mc = 8;
        while (mc > 1 && (mc / 2 >= M || (int64_t)mc * K * 4 > kRefQ4LdsBytes)) mc /= 2;
        const dim3 g4((unsigned)((N + kRows - 1) / kRows), (unsigned)((M + mc - 1) / mc), (unsigned)nslots);
        const size_t lds = (size_t)mc * (size_t)K * 4;
#define AIPU_REFREG(T)                                                                                                 \
    switch (mc) {                                                                                                      \
        case 8: hipLaunchKernelGGL((k_gemv_ref_reg<T, 8>), g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break; \
        case 4: hipLaunchKernelGGL((k_gemv_ref_reg<T, 4>), g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break; \
        case 2: hipLaunchKernelGGL((k_gemv_ref_reg<T, 2>), g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break; \
        default: hipLaunchKernelGGL((k_gemv_ref_reg<T, 1>), g4, dim3(kRows), lds, st, W, N, K, x, M, y, y_f32, ga); break; \
    }
        if (type == T_Q8_0) { AIPU_REFREG(T_Q8_0) }
        else if (type == T_F16) { AIPU_REFREG(T_F16) }
        else { AIPU_REFREG(T_BF16) }
#undef AIPU_REFREG
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((N + kRows - 1) / kRows), (unsigned)((M + kMC - 1) / kMC), (unsigned)nslots);
    switch (type) {
        case T_Q4_K: hipLaunchKernelGGL(k_gemv_ref<T_Q4_K>, grid, dim3(kRows), 0, st, W, N, K, x, M, y, y_f32, ga); break;
        case T_Q6_K: hipLaunchKernelGGL(k_gemv_ref<T_Q6_K>, grid, dim3(kRows), 0, st, W, N, K, x, M, y, y_f32, ga); break;
        case T_Q8_0: hipLaunchKernelGGL(k_gemv_ref<T_Q8_0>, grid, dim3(kRows), 0, st, W, N, K, x, M, y, y_f32, ga); break;
        case T_F16: hipLaunchKernelGGL(k_gemv_ref<T_F16>, grid, dim3(kRows), 0, st, W, N, K, x, M, y, y_f32, ga); break;
        case T_BF16: hipLaunchKernelGGL(k_gemv_ref<T_BF16>, grid, dim3(kRows), 0, st, W, N, K, x, M, y, y_f32, ga); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_ref(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                           uint16_t* y, float* y_f32, hipStream_t st) {
    return launch_gemv_ref_gather(type, w, N, K, x, M, y, y_f32, 1, nullptr, 0, 0, 0, nullptr, 0, 0, st);
}

hipError_t launch_gemv_ref_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M, uint16_t* y,
                               float* y_f32, hipStream_t st) {
    const dim3 grid((unsigned)((N + kRows - 1) / kRows), (unsigned)((M + kMC - 1) / kMC));
    hipLaunchKernelGGL(k_gemv_ref_f32, grid, dim3(kRows), 0, st, w, N, K, x, M, y, y_f32);
    return hipGetLastError();
}

}  // namespace aipu
