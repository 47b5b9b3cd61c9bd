// Streaming Q4_K GEMV building blocks for gfx950 (tolerance mode).
//
// Geometry.  A "segment" is 8 consecutive Q4_K blocks of one row (2048 weights,
// 1152 bytes).  A half-wave (32 lanes) covers one segment of one row: lane slot s = 0..31
// owns block bs = s/4 of the segment and its 64-group g = s%4, i.e. 32 bytes of qs
// (2 x 16-B loads) plus the 16-B block header (shared by the 4 lanes of the block).  The
// two halves of a wave work on two different rows ("items") with identical lane->K maps,
// so every lane's activations are fixed for the whole kernel and live in VGPRs.
//
// Arithmetic.  For a sub-block j with D = d*sc_j and Mn = dmin*m_j the reference weight is
// w = D*q - Mn.  The fast path factorises the sub-block dot product:
//     sum_k a_k w_k  ~=  D * sum_k a_k q_k  -  Mn * sum_k a_k
// sum_k a_k q_k is formed with v_dot2_f32_bf16 on biased codes: the bf16 pattern
// 0x4300 | q is exactly 128 + q for q < 16, so two codes are built with one and-or and
// the bias is removed with the per-lane constant 128 * sum_k a_k.  The products are exact
// (bf16 x small integer); only fp32 additions round, so the result is within a few ulp of
// sum|a*w| of the exact dot -- far inside the 1e-5 * sum|a*w| gate.
#pragma once

#include "common.hpp"

namespace aipu {
namespace q4f {

constexpr int kSegBlocks = 8;      // blocks per segment
constexpr int kSegWeights = 2048;  // weights per segment

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Lane constants: where the lane reads, and how its two 6-bit (scale, min) pairs are
// gathered from the 12 packed scale bytes (see q4k_pass).
struct Geo {
    int half;         // which item of the pair (lane / 32)
    int s;            // lane slot within the half, 0..31
    int bs;           // block within the segment, 0..7
    int g;            // 64-group within the block, 0..3
    uint32_t selB, selC, mC, mC4, mB2, mB;
};

__device__ __forceinline__ Geo make_geo(int lane) {
    Geo G;
    G.half = lane >> 5;
    G.s = lane & 31;
    G.bs = G.s >> 2;
    G.g = G.s & 3;
    // Sub-blocks j0 = 2g and j1 = 2g+1 both index byte jb = 2*(g&1) (+1) of their dword:
    //   g < 2 : sc_j = scales[j] & 63,  m_j = scales[j+4] & 63
    //   g >= 2: sc_j = (scales[j+4] & 15) | (scales[j-4] >> 6) << 4,
    //           m_j  = (scales[j+4] >> 4) | (scales[j]   >> 6) << 4        (ggml get_scale_min_k4)
    // B gathers [s0.b(jb), s0.b(jb+1), s1.b(jb), s1.b(jb+1)], C gathers s2's bytes jb, jb+1 twice.
    const bool lowj = G.g < 2;
    const bool jb2 = (G.g & 1) != 0;
    G.selB = jb2 ? 0x07060302u : 0x05040100u;
    G.selC = jb2 ? 0x03020302u : 0x01000100u;
    G.mC = lowj ? 0u : 0x00000F0Fu;
    G.mC4 = lowj ? 0u : 0x0F0F0000u;
    G.mB2 = lowj ? 0u : 0x30303030u;
    G.mB = lowj ? 0x3F3F3F3Fu : 0u;
    return G;
}

// Activations of one lane for one segment and one activation row: 32 bf16 pairs in the
// order the code pairs are built, plus the two sub-block sums.
struct Act {
    uint32_t xa[32];
    float alo, ahi;
};

// Build a lane's Act from 64 consecutive bf16 activations held as 32 natural-order
// dwords (a[2n] | a[2n+1] << 16), positions 64g .. 64g+63 of the lane's block.
__device__ __forceinline__ void act_from_natural(Act& A, const uint32_t (&xs)[32]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        A.xa[4 * i + 0] = perm(xs[2 * i + 1], xs[2 * i], 0x05040100u);       // a[4i],    a[4i+2]
        A.xa[4 * i + 1] = perm(xs[2 * i + 1], xs[2 * i], 0x07060302u);       // a[4i+1],  a[4i+3]
        A.xa[4 * i + 2] = perm(xs[17 + 2 * i], xs[16 + 2 * i], 0x05040100u);  // a[32+4i], a[34+4i]
        A.xa[4 * i + 3] = perm(xs[17 + 2 * i], xs[16 + 2 * i], 0x07060302u);  // a[33+4i], a[35+4i]
    }
    // sub-block sums with dot2 against (1.0, 1.0): each product is exact, fp32 adds round
    const uint32_t ones = 0x3F803F80u;
    float lo0 = 0.f, lo1 = 0.f, hi0 = 0.f, hi1 = 0.f;
#pragma unroll
    for (int n = 0; n < 16; n += 2) {
        lo0 = dot2(xs[n], ones, lo0);
        lo1 = dot2(xs[n + 1], ones, lo1);
        hi0 = dot2(xs[16 + n], ones, hi0);
        hi1 = dot2(xs[17 + n], ones, hi1);
    }
    A.alo = lo0 + lo1;
    A.ahi = hi0 + hi1;
}

__device__ __forceinline__ void act_zero(Act& A) {
#pragma unroll
    for (int i = 0; i < 32; ++i) A.xa[i] = 0u;
    A.alo = 0.f;
    A.ahi = 0.f;
}

// The 64 natural-order activations a lane owns in segment `seg` of activation row `xrow`
// (K bf16), as 32 dwords; zeros when `valid` is false.
// The loads are issued unconditionally (from `xsafe`, any 16-B aligned address with 64
// readable bf16, when !valid) and masked afterwards: a branch around them would make the
// compiler wait for every earlier vector load where the paths join.
__device__ __forceinline__ void act_load_natural(uint32_t (&xs)[32], const uint16_t* __restrict__ xrow, int seg,
                                                 const Geo& G, bool valid, const uint16_t* xsafe) {
    const int64_t k0 = (int64_t)(seg * kSegBlocks + G.bs) * QK_K + 64 * G.g;
    const uint4* p = (const uint4*)(valid ? xrow + k0 : xsafe);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint4 v = p[i];
        xs[4 * i + 0] = valid ? v.x : 0u;
        xs[4 * i + 1] = valid ? v.y : 0u;
        xs[4 * i + 2] = valid ? v.z : 0u;
        xs[4 * i + 3] = valid ? v.w : 0u;
    }
}

// Load the lane's activations for segment `seg` of activation row `xrow` (K bf16).
__device__ __forceinline__ void act_load(Act& A, const uint16_t* __restrict__ xrow, int seg, const Geo& G,
                                         bool valid) {
    uint32_t xs[32];
    act_load_natural(xs, xrow, seg, G, valid, xrow);
    act_from_natural(A, xs);
}

// Raw bytes of one lane for one item: block header + 32 bytes of qs.
struct Raw {
    uint4 h, q0, q1;
};

__device__ __forceinline__ Raw raw_load(const uint8_t* __restrict__ blk, const Geo& G) {
    const uint4* p = (const uint4*)blk;
    Raw r;
    r.h = p[0];
    r.q0 = p[1 + 2 * G.g];
    r.q1 = p[2 + 2 * G.g];
    return r;
}

// (x & 0x000F000F) | 0x43004300 in one v_bfi_b32: the two nibbles at bits 0-3 and 16-19
// become the bf16 pair (128 + n0, 128 + n1).  The constants live in registers (gfx9 VOP3
// encodings take no literals; one SGPR operand fits the constant-bus limit), so the
// select is a single VALU op.
__device__ __forceinline__ uint32_t nib2bf(uint32_t x, uint32_t mask, uint32_t bias) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(x), "v"(bias));
    return r;
}

// Sub-block dot sums of one lane: S = sum (128 + q) * a over its 32 low-nibble and 32
// high-nibble weights.
__device__ __forceinline__ void code_dots(const Raw& r, const Act& A, float& Slo, float& Shi) {
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t M = __builtin_amdgcn_readfirstlane(0x000F000Fu), B = 0x43004300u;
    float l0 = 0.f, l1 = 0.f, h0 = 0.f, h1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t x = q[i];
        const uint32_t c0 = nib2bf(x, M, B);          // bytes 0,2 low nibble
        const uint32_t c1 = nib2bf(x >> 8, M, B);     // bytes 1,3 low nibble
        const uint32_t c2 = nib2bf(x >> 4, M, B);     // bytes 0,2 high nibble
        const uint32_t c3 = nib2bf(x >> 12, M, B);    // bytes 1,3 high nibble
        l0 = dot2(A.xa[4 * i + 0], c0, l0);
        l1 = dot2(A.xa[4 * i + 1], c1, l1);
        h0 = dot2(A.xa[4 * i + 2], c2, h0);
        h1 = dot2(A.xa[4 * i + 3], c3, h1);
    }
    Slo = l0 + l1;
    Shi = h0 + h1;
}

// Header decode: d, dmin and the lane's (sc_j0, sc_j1, m_j0, m_j1) as floats.
struct Hdr {
    float d, dm, sc0, sc1, m0, m1;
};

__device__ __forceinline__ Hdr hdr_decode(const uint4& h, const Geo& G) {
    Hdr H;
    H.d = f16_to_f32(h.x);
    H.dm = f16_to_f32(h.x >> 16);
    const uint32_t B = perm(h.z, h.y, G.selB);
    const uint32_t C = perm(h.w, h.w, G.selC);
    const uint32_t R = (C & G.mC) | ((C >> 4) & G.mC4) | ((B >> 2) & G.mB2) | (B & G.mB);
    H.sc0 = (float)(R & 0xFFu);
    H.sc1 = (float)((R >> 8) & 0xFFu);
    H.m0 = (float)((R >> 16) & 0xFFu);
    H.m1 = (float)(R >> 24);
    return H;
}

// The lane's contribution to one item:  d * sum_j sc_j (S_j - 128 A_j) - dmin * sum_j m_j A_j.
__device__ __forceinline__ float lane_part(const Hdr& H, float Slo, float Shi, const Act& A) {
    const float tlo = __builtin_fmaf(-128.0f, A.alo, Slo);
    const float thi = __builtin_fmaf(-128.0f, A.ahi, Shi);
    const float u = __builtin_fmaf(H.sc1, thi, H.sc0 * tlo);
    const float v = __builtin_fmaf(H.m1, A.ahi, H.m0 * A.alo);
    return __builtin_fmaf(H.d, u, -(H.dm * v));
}

// Sum over the 32 lanes of each half-wave with DPP: quad xor 1, quad xor 2, half-row mirror,
// row mirror (each lane then holds its 16-lane row sum), and a row_bcast:15 into rows 1
// and 3.  The half-wave totals land in lanes 16..31 and 48..63.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xF, false));
}

__device__ __forceinline__ float half_sum_dpp(float v) {
    v += dpp_f<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v += dpp_f<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v += dpp_f<0x141, 0xF>(v);   // row_half_mirror
    v += dpp_f<0x140, 0xF>(v);   // row_mirror
    v += dpp_f<0x142, 0xA>(v);   // row_bcast:15 -> rows 1, 3
    return v;
}

// Sum V values across the 32 lanes of each half-wave with a transposing butterfly: the
// first log2(V) exchange steps halve the number of live values per lane, the rest are a
// plain xor tree.  Returns the total of value index (slot >> (5 - log2 V)) & (V-1).
template <int V>
__device__ __forceinline__ float half_reduce(float (&v)[V], int lane) {
    static_assert((V & (V - 1)) == 0 && V >= 1 && V <= 32, "V must be a power of two <= 32");
    constexpr int LV = V >= 32 ? 5 : V >= 16 ? 4 : V >= 8 ? 3 : V >= 4 ? 2 : V >= 2 ? 1 : 0;
#pragma unroll
    for (int i = 0, n = V; i < LV; ++i) {
        const int mask = 16 >> i;
        const bool up = (lane & mask) != 0;
        n >>= 1;
#pragma unroll
        for (int j = 0; j < V / 2; ++j) {
            if (j < n) {
                const float keep = up ? v[j + n] : v[j];
                const float send = up ? v[j] : v[j + n];
                v[j] = keep + __shfl_xor(send, mask, 64);
            }
        }
    }
    float r = v[0];
#pragma unroll
    for (int mask = 16 >> LV; mask >= 1; mask >>= 1) r += __shfl_xor(r, mask, 64);
    return r;
}

}  // namespace q4f
}  // namespace aipu
