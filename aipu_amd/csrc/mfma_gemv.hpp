// Matrix-core Q4_K GEMV core for gfx950 (tolerance mode), M = 1..4 activation rows per pass.
//
// Tile.  One wave computes a 16-row tile of the weight matrix over a range of Q4_K blocks
// with v_mfma_f32_16x16x32_bf16 (D[i][n] = sum_k A[i][k] B[k][n]; lane l supplies
// A[l%16][8(l/16)..+7] and B[8(l/16)..+7][l%16], and holds D[4(l/16)+r][l%16], r = 0..3).
//   B (weights): lane l = 16g + n owns output row n of the tile and the 32-byte qs chunk g of
//     each block (bytes 32g..32g+31), i.e. sub-block 2g in the low nibbles and sub-block
//     2g+1 in the high nibbles.  Four MFMAs (t = 0..3) cover the low nibbles, four (t = 4..7)
//     the high nibbles, 8 bytes per MFMA.
//   A (activations): block diagonal.  Row i = 4g + m of A carries activation row m (m < MR)
//     on K-group g only, so D[4g + m][n] accumulates sub-block (2g + h) of row n against
//     activation row m, for all four chunks g at once, and lane 16g + n finds exactly the
//     sums of its own row and chunk in its D registers (r = m).  All other A entries are 0.
//   Codes: a nibble q at bits 0..3 (or 16..19) of a qs dword becomes the bf16 pattern
//     0x4300 | q, which is exactly 128 + q, with one and-or per two codes (plus one shift per
//     pair not already at bits 0..3); the products (128 + q) * a are exact and the MFMA
//     accumulates in fp32.  The accumulator starts at -128 * sum(a) of the sub-block, so it
//     ends at sum(q * a).
//   Epilogue per block and lane: acc += d * (sc_lo * S_lo + sc_hi * S_hi)
//                                        - dmin * (m_lo * A_lo + m_hi * A_hi),
//     the factorised form of sum_k a_k * (d*sc*q_k - dmin*m) (tools/q4k_ref.py:53-59).
//
// Lane -> K order.  Within the 8 bytes of one MFMA the code pairs are built in byte order
// (0,2) (1,3) (4,6) (5,7); the activations are staged in LDS in the same order, so the
// products line up.  Activation piece p (8 consecutive bf16 starting at 8p) belongs to
// block p / 32, chunk (p / 8) % 4 and MFMA t = p % 8.
#pragma once

#include "common.hpp"

namespace aipu {
namespace mg {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kTR = 16;                  // output rows per tile
constexpr uint32_t kNT = 2;              // buffer-load cache policy: streaming (nt)
constexpr uint32_t kOOB = 0xF0000000u;   // buffer offset that reads as zero without a memory access
constexpr uint32_t kCodeMask = 0x000F000Fu;
constexpr uint32_t kCodeBias = 0x43004300u;   // bf16 128.0 in both halves
constexpr float kCodeBiasF = 128.0f;

__device__ __forceinline__ f32x4_t mfma(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// (v & mask) | bias in one v_and_or_b32: gfx9 VOP3 encodings take no literal and read at
// most one scalar operand, so the mask sits in an SGPR and the bias in a VGPR that the caller
// keeps live (CodeK), both hidden from constant folding (which would split the and-or into
// two literal-operand instructions).  The and-or itself is ordinary code, so the compiler's
// hazard checks see it next to the matrix instructions that read its result.
struct CodeK {
    uint32_t mask;   // wave-uniform (SGPR)
    uint32_t bias;   // VGPR
};

__device__ __forceinline__ CodeK code_k() {
    CodeK k;
    k.mask = kCodeMask;
    k.bias = kCodeBias;
    asm volatile("" : "+s"(k.mask));
    asm volatile("" : "+v"(k.bias));
    return k;
}

__device__ __forceinline__ uint32_t c16(uint32_t v, const CodeK& k) { return (v & k.mask) | k.bias; }

// B operands (128 + q codes) of the low-nibble and high-nibble MFMAs over qs dwords x0, x1:
// element pairs (byte 0, byte 2), (1, 3), (4, 6), (5, 7) of the 8 bytes.
__device__ __forceinline__ u32x4_t codes_lo(uint32_t x0, uint32_t x1, const CodeK& k) {
    return u32x4_t{c16(x0, k), c16(x0 >> 8, k), c16(x1, k), c16(x1 >> 8, k)};
}
__device__ __forceinline__ u32x4_t codes_hi(uint32_t x0, uint32_t x1, const CodeK& k) {
    return u32x4_t{c16(x0 >> 4, k), c16(x0 >> 12, k), c16(x1 >> 4, k), c16(x1 >> 12, k)};
}

// 8 natural-order bf16 (w0 = a0|a1<<16 ...) -> the MFMA element order (a0,a2)(a1,a3)(a4,a6)(a5,a7).
__device__ __forceinline__ u32x4_t act_perm(const uint4& v) {
    return u32x4_t{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                   __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
}

__device__ __forceinline__ uint4 wload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// One lane's bytes of one block: the 16-B header and its 32-B qs chunk.
struct Raw {
    uint4 h, q0, q1;
};

__device__ __forceinline__ Raw raw_load(__amdgpu_buffer_rsrc_t r, uint32_t off, int g) {
    Raw x;
    x.h = wload(r, off);
    x.q0 = wload(r, off + 16u + 32u * g);
    x.q1 = wload(r, off + 32u + 32u * g);
    return x;
}

// Scale/min of sub-blocks 2g and 2g+1 from the 12 packed bytes (header dwords y, z, w),
// following get_scale_min_k4 (tools/q4k_ref.py:27-37):
//   j < 4 : sc = s[j] & 63,                      m = s[j+4] & 63
//   j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4,  m = (s[j+4] >> 4) | (s[j] >> 6) << 4
// Sub-blocks 2g, 2g+1 read bytes jb = 2(g&1), jb+1 of each dword.
struct HdrSel {
    uint32_t selB, selC, mC, mC4, mB2, mB;
};

__device__ __forceinline__ HdrSel hdr_sel(int g) {
    HdrSel s;
    const bool lowj = g < 2;
    const bool jb2 = (g & 1) != 0;
    s.selB = jb2 ? 0x07060302u : 0x05040100u;
    s.selC = jb2 ? 0x03020302u : 0x01000100u;
    s.mC = lowj ? 0u : 0x00000F0Fu;
    s.mC4 = lowj ? 0u : 0x0F0F0000u;
    s.mB2 = lowj ? 0u : 0x30303030u;
    s.mB = lowj ? 0x3F3F3F3Fu : 0u;
    return s;
}

struct Hdr {
    float d, dm, sc0, sc1, m0, m1;
};

__device__ __forceinline__ Hdr hdr_decode(const uint4& h, const HdrSel& S) {
    Hdr H;
    H.d = f16_to_f32(h.x);
    H.dm = f16_to_f32(h.x >> 16);
    const uint32_t B = __builtin_amdgcn_perm(h.z, h.y, S.selB);
    const uint32_t C = __builtin_amdgcn_perm(h.w, h.w, S.selC);
    const uint32_t R = (C & S.mC) | ((C >> 4) & S.mC4) | ((B >> 2) & S.mB2) | (B & S.mB);
    H.sc0 = (float)(R & 0xFFu);
    H.sc1 = (float)((R >> 8) & 0xFFu);
    H.m0 = (float)((R >> 16) & 0xFFu);
    H.m1 = (float)(R >> 24);
    return H;
}

// One Q4_K block of a 16-row tile against one activation row, on lane 16g + n: the eight
// MFMAs over the biased codes (accumulators seeded with -128 * the sub-block activation
// sums `as`), then the scale/min epilogue.  A holds the block's activation operands (only
// the diagonal lanes nonzero); dlo / dhi keep their off-diagonal entries at zero.
__device__ __forceinline__ float q4k_block1(const Raw& R, const u32x4_t (&A)[8], float2 as, const HdrSel& hs,
                                            const CodeK& ck, f32x4_t& dlo, f32x4_t& dhi, float acc) {
    dlo[0] = -kCodeBiasF * as.x;
    dhi[0] = -kCodeBiasF * as.y;
    const uint32_t qd[8] = {R.q0.x, R.q0.y, R.q0.z, R.q0.w, R.q1.x, R.q1.y, R.q1.z, R.q1.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        dlo = mfma(A[t], codes_lo(qd[2 * t], qd[2 * t + 1], ck), dlo);
        dhi = mfma(A[4 + t], codes_hi(qd[2 * t], qd[2 * t + 1], ck), dhi);
    }
    const Hdr H = hdr_decode(R.h, hs);
    const float t1 = __builtin_fmaf(H.sc1, dhi[0], H.sc0 * dlo[0]);
    const float v = __builtin_fmaf(H.m1, as.y, H.m0 * as.x);
    acc = __builtin_fmaf(H.d, t1, acc);
    return __builtin_fmaf(-H.dm, v, acc);
}

// ------------------------------------------------------------- LDS helpers

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// The 8 activation operands of a block, read on the lanes in `mask` only (the diagonal
// lanes of the block-diagonal A); every other lane keeps its register contents, which stay
// zero for the whole kernel.  This moves 64 B per read instead of a 1 KB broadcast of zeros.
// The loads complete inside the asm (lgkmcnt(0) before it returns): the compiler treats the
// outputs as written when the statement ends, so no load may still be in flight then.
// s_and_b64 sets SCC, so SCC is declared clobbered (the compiler may keep a loop condition
// there).
__device__ __forceinline__ void a_reads(u32x4_t (&A)[8], uint32_t aa, uint64_t mask) {
    uint64_t saved;
    asm volatile(
        "s_mov_b64 %8, exec\n\t"
        "s_and_b64 exec, exec, %10\n\t"
        "ds_read_b128 %0, %9\n\t"
        "ds_read_b128 %1, %9 offset:64\n\t"
        "ds_read_b128 %2, %9 offset:128\n\t"
        "ds_read_b128 %3, %9 offset:192\n\t"
        "ds_read_b128 %4, %9 offset:256\n\t"
        "ds_read_b128 %5, %9 offset:320\n\t"
        "ds_read_b128 %6, %9 offset:384\n\t"
        "ds_read_b128 %7, %9 offset:448\n\t"
        "s_mov_b64 exec, %8\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(A[3]), "+v"(A[4]), "+v"(A[5]), "+v"(A[6]), "+v"(A[7]),
          "=&s"(saved)
        : "v"(aa), "s"(mask)
        : "memory", "scc");   // s_and_b64 writes SCC
}

// Half of a_reads for a pair-major layout: the operands of four MFMAs, 128 B apart (entries
// [t][g][m], m < 2, per pair).
__device__ __forceinline__ void a_reads2h(u32x4_t (&A)[4], uint32_t aa, uint64_t mask) {
    uint64_t saved;
    asm volatile(
        "s_mov_b64 %4, exec\n\t"
        "s_and_b64 exec, exec, %6\n\t"
        "ds_read_b128 %0, %5\n\t"
        "ds_read_b128 %1, %5 offset:128\n\t"
        "ds_read_b128 %2, %5 offset:256\n\t"
        "ds_read_b128 %3, %5 offset:384\n\t"
        "s_mov_b64 exec, %4\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(A[3]), "=&s"(saved)
        : "v"(aa), "s"(mask)
        : "memory", "scc");
}

// A point after which the weight blocks in R are in registers: the asm consumes every
// register of R (so the LDS loads that produce them have completed), and its memory clobber
// keeps later memory operations -- the copy that refills the same LDS slice -- behind it.
template <class T, int N>
__device__ __forceinline__ void regs_consumed(const T (&R)[N]) {
    static_assert(sizeof(T) % 4 == 0, "register blocks are whole dwords");
    struct Dw {
        uint32_t d[sizeof(T) / 4];
    };
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const Dw w = __builtin_bit_cast(Dw, R[i]);
#pragma unroll
        for (int k = 0; k < (int)(sizeof(T) / 4); ++k) asm volatile("" ::"v"(w.d[k]) : "memory");
    }
}

// The sub-block activation sums (lo, hi) of one block for this lane, read inside an asm
// statement that also waits for it: the compiler sees no LDS load there, so it does not
// order the read behind direct-to-LDS copies still in flight into other LDS buffers.
__device__ __forceinline__ float2 sums_read(const float* p) {
    float2 v;
    asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
    return v;
}


// Diagonal lanes of the block-diagonal activation operand: lane 16g + 4g + m for m < MR.
__host__ __device__ constexpr uint64_t diag_mask(int mr) {
    uint64_t m = 0;
    for (int g = 0; g < 4; ++g)
        for (int r = 0; r < mr; ++r) m |= 1ull << (20 * g + r);
    return m;
}

template <uint32_t POL = kNT>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, POL);
}

// s_waitcnt immediates (gfx9 layout: vmcnt[3:0] expcnt[6:4] lgkmcnt[11:8] vmcnt_hi[15:14])
constexpr int kWaitVm0 = 0x0F70;    // vmcnt(0)
constexpr int kWaitLgkm0 = 0xC07F;  // lgkmcnt(0)
// s_waitcnt immediate for vmcnt(n), n < 64 (vmcnt bits 3:0 and 15:14)
__host__ __device__ constexpr int wait_vm(int n) { return (kWaitVm0 & ~0xC00F) | (n & 0x0F) | ((n >> 4) << 14); }

// LDS layout of one staged activation (M_pad = MR rows, nsb blocks):
//   A entries (16 B): [b][t][g][m]  at index (b*8 + t)*4*MR + g*MR + m
//   sums (fp32):      [b][g][h][m]  at index ((b*4 + g)*2 + h)*MR + m
// and a zero region of 8*4*MR entries that the off-diagonal lanes read.
template <int MR>
struct ActLayout {
    static constexpr int kEntriesPerBlock = 8 * 4 * MR;
    static constexpr int kSumsPerBlock = 8 * MR;
    __host__ __device__ static int64_t bytes(int nsb) { return (int64_t)nsb * (kEntriesPerBlock * 16 + kSumsPerBlock * 4); }
    static constexpr int kZeroBytes = kEntriesPerBlock * 16;
};

// ------------------------------------------------------------- fast-mode reduction order
// The single-row kernels and the small-batch kernels (k_gemvs, k_gemvm) of the tolerance mode
// form an output the same way, so a row of a batch they serve equals the single-row result bit
// for bit (the persistent multi-row kernel uses its own, dense form):
//   1. per block b and K-group g (lane 16g + n): S_lo, S_hi from the MFMA chain (seeded with
//      -128 * the sub-block activation sums), then
//         term_g = fma(-dmin, fma(m1, A_hi, m0 * A_lo), d * fma(sc1, S_hi, sc0 * S_lo));
//   2. block term B_b = (term_0 + term_1) + (term_2 + term_3)       (block_sum)
//   3. pair sums s_p = B_2p + B_2p+1 (B_nsb = 0 for odd nsb);
//   4. v_k = s_k + s_k+8 + s_k+16 + ... (left to right; v_k = 0 for k >= #pairs), k < 8;
//   5. y = ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)).
// Steps 3-5 are a balanced tree over the pairs that a wave-per-pair kernel evaluates with
// three cross-lane adds and a kernel holding all block terms evaluates with canon_sum.

__device__ __forceinline__ float block_term(const Hdr& H, float slo, float shi, float alo, float ahi) {
    const float t1 = __builtin_fmaf(H.sc1, shi, H.sc0 * slo);
    const float v = __builtin_fmaf(H.m1, ahi, H.m0 * alo);
    return __builtin_fmaf(-H.dm, v, H.d * t1);
}

// Sum over the four K-groups (lanes n, n + 16, n + 32, n + 48), in every lane.
__device__ __forceinline__ float block_sum(float a) {
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    const float s = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

// block_sum of four values at once, transposed: lane 16i + n returns a_i's sum over the lanes
// n, n + 16, n + 32, n + 48.  permlane16_swap(X, Y) swaps X's odd 16-lane rows with Y's even
// rows, so X + Y holds (g0 + g1) of X, Y, X, Y in rows 0..3 ... of (X, Y) = (a0, a1), and
// (g2 + g3) in rows 2, 3; permlane32_swap then pairs each (g0 + g1) with its (g2 + g3).  The
// additions are those of block_sum, so the bits are too.
__device__ __forceinline__ float block_sum4(float a0, float a1, float a2, float a3) {
    const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(a0), __float_as_uint(a1), false, false);
    const auto y = __builtin_amdgcn_permlane16_swap(__float_as_uint(a2), __float_as_uint(a3), false, false);
    const float s01 = __uint_as_float(x[0]) + __uint_as_float(x[1]);   // rows: a0 g01, a1 g01, a0 g23, a1 g23
    const float s23 = __uint_as_float(y[0]) + __uint_as_float(y[1]);   // rows: a2 g01, a3 g01, a2 g23, a3 g23
    const auto z = __builtin_amdgcn_permlane32_swap(__float_as_uint(s01), __float_as_uint(s23), false, false);
    return __uint_as_float(z[0]) + __uint_as_float(z[1]);               // rows: a0, a1, a2, a3
}
// Two values: lane 16i + n returns a_(i & 1)'s sum.
__device__ __forceinline__ float block_sum2(float a0, float a1) {
    const auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(a0), __float_as_uint(a1), false, false);
    const float s = __uint_as_float(x[0]) + __uint_as_float(x[1]);     // rows: a0 g01, a1 g01, a0 g23, a1 g23
    const auto z = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(z[0]) + __uint_as_float(z[1]);               // rows: a0, a1, a0, a1
}

// Steps 3-5 over block terms bt(b), b < nsb.
template <class F>
__device__ __forceinline__ float canon_sum(int nsb, F&& bt) {
    const int np = (nsb + 1) >> 1;
    auto pair = [&](int p) { return bt(2 * p) + (2 * p + 1 < nsb ? bt(2 * p + 1) : 0.0f); };
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        v[k] = k < np ? pair(k) : 0.0f;
        for (int i = k + 8; i < np; i += 8) v[k] += pair(i);
    }
    return ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
}

// The same sum on eight lanes (k = lane & 7 of an aligned group of eight, all lanes active):
// lane k forms v_k, then xor 1, xor 2 and the half-row mirror add the tree; every lane of the
// group ends with y.  Bit-identical to canon_sum (IEEE addition commutes).
template <class F>
__device__ __forceinline__ float canon_sum8(int nsb, int k, F&& bt) {
    const int np = (nsb + 1) >> 1;
    auto pair = [&](int p) { return bt(2 * p) + (2 * p + 1 < nsb ? bt(2 * p + 1) : 0.0f); };
    float v = k < np ? pair(k) : 0.0f;
    for (int i = k + 8; i < np; i += 8) v += pair(i);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));    // xor 1
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));    // xor 2
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));   // half-row mirror
    return v;
}

}  // namespace mg
}  // namespace aipu
