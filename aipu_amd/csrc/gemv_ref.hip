// Reference-order GEMV: bit-identical to the reference's golden for every ggml type.
//
// Contract (tools/q4k_ref.py:67-92, RTL order src/glm_matmul_q4k.v:261-270): for each
// output (m, n) the weight row is dequantised exactly and
//     acc = f32(acc + f32(x[m][k] * w[n][k]))     for k = 0 .. K-1, in order,
// then y = bf16_RNE(acc).  One lane owns one output row and walks K sequentially; the
// 64 rows of a workgroup are staged 256 weights at a time through LDS so the global
// reads stay coalesced.  A last stage of fewer weights serves K that is a multiple of the
// type's block but not of 256 (Q8_0: 32; F16 / BF16: any K).  The library is compiled with -ffp-contract=off, so the multiply
// and the add below are two separately rounded ops.
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
    const dim3 grid((unsigned)((N + kRows - 1) / kRows), (unsigned)((M + kMC - 1) / kMC), (unsigned)nslots);
    const uint8_t* W = (const uint8_t*)w;
    const RefGather ga{sel, topk, E, wstride, (const uint8_t*)w_alt, x_zstride, y_zstride};
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
