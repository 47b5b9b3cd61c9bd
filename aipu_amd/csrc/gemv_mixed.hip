// Mixed-type GEMV (tolerance mode, MR <= 4 activation rows per launch): one launch over a list of tiles,
// each a run of output rows stored as Q4_K, Q6_K, Q8_0, F16 or BF16 -- the per-column
// w_type mux of src/glm_matmul_q4k.v:76-101,197-259 over the tile sequence of
// tools/q4k_mixed_gen.py:382-440.  A single-tile call serves the plain GEMV of Q6_K, Q8_0 and F16.
//
// Workgroup.  Four waves own one 16-row group of one tile; wave w takes the w-th quarter of the
// row's 256-weight blocks.  Each wave stages its own activations, then streams its 16 rows group
// by group (GS blocks per group) into its own LDS slice with direct-to-LDS buffer loads (16
// consecutive bytes per lane, so one instruction covers ~1 KB of row bytes), and copies a group
// into registers before the next group's loads are issued into the slice.  The four parts are
// added in fixed order, so results are deterministic.
//
// Arithmetic.  Every type runs on the matrix cores with the block-diagonal activation operand of
// mfma_gemv.hpp: lane 16g + n supplies 8 weights of output row n on K-group g of an MFMA, row
// 4g + m of the activation operand carries activation row m on K-group g only, and D register m
// of lane 16g + n accumulates row m's products for that weight row and K-group.  One MFMA thus
// serves every activation row of the launch, each row's sums are formed exactly as in a one-row
// launch (the rows of a batch equal their single-row results bit for bit), and the weights are
// read and turned into operands once per launch.  Each type's weights become exact operands:
//   Q4_K: the biased codes of mfma_gemv.hpp (bf16 128 + q, chains seeded with -128 * sum a);
//   Q6_K (tools/q4k_ref.py:105-124): the 6-bit code c as bf16 128 + c (0x4300 | c); a chain of
//        two MFMAs per 16-weight scale group, seeded with -160 * the group's activation sum,
//        ends at sum a (c - 32), then acc += f32(d * sc) * chain;
//   Q8_0 (tools/q4k_ref.py:126-129): q + 128 = byte ^ 0x80 as fp16 1024 + q + 128 (0x6400 | byte);
//        a chain of four MFMAs per 32-weight block, seeded with -1152 * sum a, ends at sum a q,
//        then acc += d * chain;
//   F16 / BF16 (tools/glm_model_q4k_ref.py:61-63): the weights themselves, one chain per part.
// bf16 operands (Q4_K, Q6_K, BF16) take the activations as they are.  fp16 operands (Q8_0, F16)
// take them scaled by 2^-e, e per activation row and wave, chosen so that the largest magnitude
// of the wave's part lies in [2^14, 2^15): every bf16 value down to 2^-31 of that maximum
// converts exactly and smaller ones lose at most 2^-25 * 2^e; the part's sum is scaled back by
// 2^e.  All products are exact; the matrix cores add them in fp32.  The order of additions
// differs from the reference's sequential MAC, so this is the tolerance path; the
// reference-order kernel (gemv_ref.hip) is the bit-exact one.
#include "common.hpp"
#include "launch.hpp"
#include "mfma_gemv.hpp"

#include <type_traits>

namespace aipu {

using namespace mg;

namespace {

constexpr int kMixW = 4;                  // waves per workgroup (= K parts)
constexpr int kSliceBytes = 9 * 1024;     // per-wave weight slice: the largest group below

// Bytes of one 256-weight block of one row in memory (kBlk) and in the LDS slice (kPitch),
// and blocks per streamed group (GS) of 16 rows.  A Q6_K block is copied as 14 whole 16-B
// pieces (224 bytes of LDS) so that every block starts 16-B aligned: pieces 0..12 are bytes
// 0..207 and piece 13 is bytes 194..209, so no piece reaches past the block (d lands at LDS
// byte 222).  Q8_0 "blocks" are runs of eight 34-B ggml blocks.
template <int TYPE>
struct Geom;
template <>
struct Geom<T_Q4_K> {
    static constexpr int kBlk = 144, kPitch = 144, GS = 3;
};
template <>
struct Geom<T_Q6_K> {
    static constexpr int kBlk = 210, kPitch = 224, GS = 2;
};
template <>
struct Geom<T_Q8_0> {
    static constexpr int kBlk = 272, kPitch = 272, GS = 2;
};
template <>
struct Geom<T_F16> {
    static constexpr int kBlk = 512, kPitch = 512, GS = 1;
};
template <>
struct Geom<T_BF16> {
    static constexpr int kBlk = 512, kPitch = 512, GS = 1;
};

// Direct-to-LDS copy of one group: piece j (16 B) of the slice is piece p of block b of row
// r, j = (r * GS + b) * kPitch / 16 + p.  Lanes past the last piece, and blocks past the
// wave's range, read through the out-of-range offset (zeros, no memory access).
template <int TYPE>
struct MixDma {
    typedef Geom<TYPE> G;
    static constexpr int kP16 = G::kPitch / 16;
    static constexpr int kRowPieces = G::GS * kP16;
    static constexpr int kPieces = kTR * kRowPieces;
    static constexpr int kInsts = (kPieces + 63) / 64;
    static_assert(kInsts * 1024 <= kSliceBytes, "slice too small");
    uint32_t off[kInsts];
    int blk[kInsts];
    __device__ void init(int lane, int64_t rb) {
#pragma unroll
        for (int i = 0; i < kInsts; ++i) {
            const int j = 64 * i + lane;
            const int r = j / kRowPieces, rem = j - r * kRowPieces;
            const int b = rem / kP16, p = rem - b * kP16;
            const int src = 16 * p < G::kBlk - 16 ? 16 * p : G::kBlk - 16;   // the last piece ends at the block's end
            off[i] = (uint32_t)(r * rb) + (uint32_t)(b * G::kBlk + src);
            blk[i] = j < kPieces ? b : G::GS;
        }
    }
    __device__ void issue(__amdgpu_buffer_rsrc_t wr, uint8_t* slice, int b0, int nb) const {
#pragma unroll
        for (int i = 0; i < kInsts; ++i) {
            const uint32_t o = blk[i] < nb ? off[i] + (uint32_t)(b0 * G::kBlk) : kOOB;
            lds_dma16(wr, slice + 1024 * i, o);
        }
    }
};

// ---------------------------------------------------------------- operands
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4_t mfma_h(const u32x4_t& a, const u32x4_t& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0,
                                                  0, 0);
}

// Bytes 0, 1 (or 2, 3) of v as two 16-bit operands (hb << 8) | byte, hb the byte in every byte of k:
// with hb = 0x43 the bf16 value 128 + byte (byte < 128), with hb = 0x64 the fp16 value 1024 + byte.
__device__ __forceinline__ uint32_t bytes01(uint32_t v, uint32_t k) { return __builtin_amdgcn_perm(k, v, 0x04010400u); }
__device__ __forceinline__ uint32_t bytes23(uint32_t v, uint32_t k) { return __builtin_amdgcn_perm(k, v, 0x04030402u); }

// The exponent e that puts the largest |x| of a wave's part (mx = its bf16 magnitude bits)
// times 2^-e in [2^14, 2^15); 0 for an all-zero part or one holding inf / nan.
__device__ __forceinline__ int part_exponent(uint32_t mx) {
    if (mx == 0 || mx >= 0x7F80u) return 0;
    int ex;
    (void)frexpf(bf16_to_f32(mx), &ex);   // max = f * 2^ex, f in [0.5, 1)
    return ex - 15;
}

// Two bf16 (one dword) times 2^-e as an fp16 pair, round to nearest even.
__device__ __forceinline__ uint32_t f16_pair_scaled(uint32_t w, int e) {
    const float lo = __builtin_ldexpf(__uint_as_float(w << 16), -e);
    const float hi = __builtin_ldexpf(__uint_as_float(w & 0xFFFF0000u), -e);
    return (uint32_t)__half_as_ushort(__float2half_rn(lo)) | ((uint32_t)__half_as_ushort(__float2half_rn(hi)) << 16);
}

// ---------------------------------------------------------------- per-type blocks
// Q6_K: the lane's bytes of one block (ql runs at 64h + o and 64h + 32 + o, qh at
// 128 + 32h + o, the 8 scales of half h, d), h = g >> 1, o = 16 (g & 1).
struct RawQ6 {
    uint4 ql0, ql1, qh;
    uint2 sc;
    uint32_t d;   // fp16 bits
};

__device__ __forceinline__ RawQ6 q6_read(const uint8_t* blk, int g) {
    const int h = g >> 1, o = 16 * (g & 1);
    RawQ6 r;
    r.ql0 = *(const uint4*)(blk + 64 * h + o);
    r.ql1 = *(const uint4*)(blk + 64 * h + 32 + o);
    r.qh = *(const uint4*)(blk + 128 + 32 * h + o);
    r.sc = *(const uint2*)(blk + 192 + 8 * h);
    r.d = *(const uint16_t*)(blk + 222);   // block bytes 208..209 (see Geom<T_Q6_K>)
    return r;
}

// Q8_0: the lane's two 34-B blocks (2g, 2g+1 of the run of eight): 17 dwords.
struct RawQ8 {
    uint32_t w[17];
};

__device__ __forceinline__ RawQ8 q8_read(const uint8_t* run, int g) {
    const uint32_t* p = (const uint32_t*)(run + 68 * g);
    RawQ8 r;
#pragma unroll
    for (int k = 0; k < 17; ++k) r.w[k] = p[k];
    return r;
}

// F16 / BF16: the lane's 64 weights (128 B).
struct Raw128 {
    uint4 v[8];
};

// One Q4_K block for MR rows: the eight MFMAs of mfma_gemv.hpp with row m's seeds in D
// register m, then row m's scale/min epilogue -- q4k_block1 with D register 0 replaced by m.
template <int MR>
__device__ __forceinline__ void q4k_block_rows(const Raw& R, const u32x4_t (&A)[8], const float2 (&as)[MR],
                                               const HdrSel& hs, const CodeK& ck, float (&acc)[MR]) {
    f32x4_t dlo = {0.f, 0.f, 0.f, 0.f}, dhi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        dlo[m] = -kCodeBiasF * as[m].x;
        dhi[m] = -kCodeBiasF * as[m].y;
    }
    const uint32_t qd[8] = {R.q0.x, R.q0.y, R.q0.z, R.q0.w, R.q1.x, R.q1.y, R.q1.z, R.q1.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        dlo = mfma(A[t], codes_lo(qd[2 * t], qd[2 * t + 1], ck), dlo);
        dhi = mfma(A[4 + t], codes_hi(qd[2 * t], qd[2 * t + 1], ck), dhi);
    }
    const Hdr H = hdr_decode(R.h, hs);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const float t1 = __builtin_fmaf(H.sc1, dhi[m], H.sc0 * dlo[m]);
        const float v = __builtin_fmaf(H.m1, as[m].y, H.m0 * as[m].x);
        acc[m] = __builtin_fmaf(H.d, t1, acc[m]);
        acc[m] = __builtin_fmaf(-H.dm, v, acc[m]);
    }
}

// One Q6_K block for MR rows on lane 16g + n.  Position 128h + 32t + l takes the low (t < 2)
// or high nibble of ql[64h + 32(t&1) + l] and bits 2t..2t+1 of qh[32h + l]; the lane's l run
// over o..o+15, scale index 8h + 2t + (g & 1).  MFMA 2t + j covers l = o + 8j .. o + 8j + 7;
// sg[m][t] is row m's activation sum over the lane's 16 positions of run t.
template <int MR>
__device__ __forceinline__ void q6_block_rows(const RawQ6& r, const u32x4_t (&A)[8], const float4 (&sg)[MR], int g,
                                              float (&acc)[MR]) {
    const uint32_t kb = 0x43434343u;
    const uint32_t ql0[4] = {r.ql0.x, r.ql0.y, r.ql0.z, r.ql0.w};
    const uint32_t ql1[4] = {r.ql1.x, r.ql1.y, r.ql1.z, r.ql1.w};
    const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    f32x4_t D[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        D[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < MR; ++m) D[t][m] = -160.0f * (t == 0 ? sg[m].x : t == 1 ? sg[m].y : t == 2 ? sg[m].z : sg[m].w);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            uint32_t c[2];
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int k = 2 * j + kk;
                const uint32_t ql = t & 1 ? ql1[k] : ql0[k];
                const uint32_t nib = (t < 2 ? ql : ql >> 4) & 0x0F0F0F0Fu;
                const uint32_t hb = t == 0 ? qh[k] << 4 : t == 1 ? qh[k] << 2 : t == 2 ? qh[k] : qh[k] >> 2;
                c[kk] = nib | (hb & 0x30303030u);
            }
            D[t] = mfma(A[2 * t + j], u32x4_t{bytes01(c[0], kb), bytes23(c[0], kb), bytes01(c[1], kb), bytes23(c[1], kb)},
                        D[t]);
        }
    const float d = f16_to_f32(r.d);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int sci = (g & 1) + 2 * t;   // byte of the half's 8 scales
        const uint32_t scw = sci < 4 ? r.sc.x : r.sc.y;
        const float dsc = d * (float)(int)(int8_t)(uint8_t)(scw >> (8 * (sci & 3)));
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = __builtin_fmaf(dsc, D[t][m], acc[m]);
    }
}

// One run of eight Q8_0 blocks for MR rows on lane 16g + n: ggml blocks 2g (codes at bytes
// 2..33 of the lane's 68) and 2g + 1 (bytes 36..67); MFMA s < 4 covers codes 8s..8s+7 of the
// first, s >= 4 codes 8(s-4).. of the second.  s32[m] holds row m's sums of the two blocks'
// scaled activations.
template <int MR>
__device__ __forceinline__ void q8_block_rows(const RawQ8& r, const u32x4_t (&A)[8], const float2 (&s32)[MR],
                                              float (&acc)[MR]) {
    const uint32_t kh = 0x64646464u;
    uint32_t x[17];
#pragma unroll
    for (int k = 0; k < 17; ++k) x[k] = r.w[k] ^ 0x80808080u;   // bytes -> q + 128
    f32x4_t D0 = {0.f, 0.f, 0.f, 0.f}, D1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        D0[m] = -1152.0f * s32[m].x;
        D1[m] = -1152.0f * s32[m].y;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        D0 = mfma_h(A[s], u32x4_t{bytes23(x[2 * s], kh), bytes01(x[2 * s + 1], kh), bytes23(x[2 * s + 1], kh),
                                  bytes01(x[2 * s + 2], kh)},
                    D0);
        D1 = mfma_h(A[4 + s], u32x4_t{bytes01(x[9 + 2 * s], kh), bytes23(x[9 + 2 * s], kh), bytes01(x[10 + 2 * s], kh),
                                      bytes23(x[10 + 2 * s], kh)},
                    D1);
    }
    const float d0 = f16_to_f32(r.w[0]), d1 = f16_to_f32(r.w[8] >> 16);
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        acc[m] = __builtin_fmaf(d0, D0[m], acc[m]);
        acc[m] = __builtin_fmaf(d1, D1[m], acc[m]);
    }
}

// ------------------------------------------------------------------ kernel
struct MixTile {
    const uint8_t* w;
    int64_t row0;
    int32_t nrows, type;
    int32_t wg0, pad;   // first workgroup of the tile
};

// Tiles in workgroup order (heaviest row bytes first); workgroups past the first `split` take
// the groups from the end backwards (see launch_gemv_mixed).
struct MixArgs {
    MixTile t[AIPU_MAX_TILES];
    int n, nwg, split;
};

// Per-wave activation region of one row: a ring of four block slots, block b in slot b % 4.
// A slot holds the operand entries [8 MFMAs][4 K-groups] of 16 B (512 B per block), and the
// slots' sums that the type's chains are seeded with follow (Q4_K: 8 sub-block sums per block
// [slot][g][h]; Q6_K: 16 sums of 16 [slot][g][t]; Q8_0: 8 block sums [slot][2g + c]).
// Entry (b, s, g) holds the 8 activations that lane group g multiplies in MFMA s of block b:
//   Q4_K: pieces 32b + 8g + s in the element order of mfma_gemv.hpp (act_perm);
//   Q6_K: positions 128(g>>1) + 32(s>>1) + 16(g&1) + 8(s&1) + e, e = 0..7;
//   Q8_0, F16, BF16: positions 64g + 8s + e;
// fp16 (scaled) for Q8_0 and F16, bf16 otherwise.  A wave stages blocks 0..3 of its part
// before its first group and blocks 2i, 2i + 1 (i >= 2) into the slots of blocks 2i - 4,
// 2i - 3 just before the first group that needs them; groups of at most three blocks run in
// order, so those blocks have been used by then.  Four slots per row, not the whole part,
// keep four rows and the weight slices within half the CU's LDS: two workgroups share a CU.
constexpr int kRing = 4;
struct ActRegion {
    static constexpr int kBytes = kRing * (512 + 64);
    static constexpr int kSumOff = kRing * 512;
};

template <int TYPE, int XI, int MR>
__device__ __forceinline__ void mix_body(const MixTile& T, int grp, const uint16_t* __restrict__ X, int K, int M,
                                         uint8_t* wA, uint8_t* wW, float* red, uint16_t* Y, float* Yf, int64_t ys) {
    typedef Geom<TYPE> G;
    typedef ActRegion AR;
    static_assert(G::GS <= 3, "a group must not reach back to the slots it restages");
    constexpr bool kHalf = TYPE == T_Q8_0 || TYPE == T_F16;   // fp16 operands, scaled activations
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nsb = K / QK_K;
    const int kb0 = w * nsb / kMixW, kb1 = (w + 1) * nsb / kMixW;
    const int bpk = kb1 - kb0;
    const int NG = (bpk + G::GS - 1) / G::GS;
    const int64_t rb = (int64_t)nsb * G::kBlk;
    const int r0 = grp * kTR;
    const int nvalid = T.nrows - r0 < kTR ? T.nrows - r0 : kTR;

    // 1. this wave's activations of every row (pieces past its blocks, and rows past M, read
    // as zero), 2. its first group
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, (uint32_t)(M * K) * 2u);
    const uint32_t xbase = 2u * (uint32_t)(kb0 * QK_K);
    const int XP = bpk * 32;
    uint4 xv[MR][XI];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const int q = lane + 64 * i;
            xv[m][i] = buf_load16(xr, q < XP && m < M ? 2u * (uint32_t)(m * K) + xbase + 16u * q : kOOB);
        }
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(T.w + (int64_t)r0 * rb, (uint32_t)(nvalid * rb));
    MixDma<TYPE> dma;
    dma.init(lane, rb);
    dma.issue(wr, wW, kb0, bpk < G::GS ? bpk : G::GS);
    __builtin_amdgcn_sched_barrier(0);

    // 3. the row exponents (fp16 operands), then stage blocks 0..3 (every piece, so blocks past
    // bpk hold zeros); row m at m * kBytes
    int ex[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        ex[m] = 0;
        if constexpr (kHalf) {
            uint32_t mx = 0;
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const uint32_t v[4] = {xv[m][i].x, xv[m][i].y, xv[m][i].z, xv[m][i].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) mx = max(mx, max(v[k] & 0x7FFFu, (v[k] >> 16) & 0x7FFFu));
            }
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, s, 64));
            ex[m] = part_exponent(mx);
        }
    }
    // pieces q = lane + 64 i (blocks 2i, 2i + 1) of every row into their ring slots
    auto stage = [&](int i) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            uint8_t* rA = wA + m * AR::kBytes;
            float* wS = (float*)(rA + AR::kSumOff);
            const int q = lane + 64 * i, bb = (q >> 5) & (kRing - 1), qq = q & 31;
            if constexpr (TYPE == T_Q4_K) {
                const uint32_t ones = 0x3F803F80u;
                float sm = 0.f;
                sm = dot2(xv[m][i].x, ones, sm);
                sm = dot2(xv[m][i].y, ones, sm);
                sm = dot2(xv[m][i].z, ones, sm);
                sm = dot2(xv[m][i].w, ones, sm);
                sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
                sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x4E, 0xF, 0xF, false));
                const int gg = (q >> 3) & 3, t = q & 7;
                *(u32x4_t*)(rA + 16u * (uint32_t)((bb * 8 + t) * 4 + gg)) = act_perm(xv[m][i]);
                if ((q & 3) == 0) wS[(bb * 4 + gg) * 2 + ((q >> 2) & 1)] = sm;
            } else if constexpr (TYPE == T_Q6_K) {
                const int h = qq >> 4, t = (qq >> 2) & 3, gl = (qq >> 1) & 1, j = qq & 1;
                const int gq = 2 * h + gl;
                *(uint4*)(rA + 16u * (uint32_t)((bb * 8 + 2 * t + j) * 4 + gq)) = xv[m][i];
                const uint32_t v[4] = {xv[m][i].x, xv[m][i].y, xv[m][i].z, xv[m][i].w};
                float f[8];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    f[2 * k] = __uint_as_float(v[k] << 16);
                    f[2 * k + 1] = __uint_as_float(v[k] & 0xFFFF0000u);
                }
                float sm = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
                sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
                if (j == 0) wS[16 * bb + 4 * gq + t] = sm;
            } else if constexpr (TYPE == T_BF16) {
                *(uint4*)(rA + 16u * (uint32_t)((bb * 8 + (qq & 7)) * 4 + (qq >> 3))) = xv[m][i];
            } else {
                const uint32_t v[4] = {xv[m][i].x, xv[m][i].y, xv[m][i].z, xv[m][i].w};
                uint32_t hv[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) hv[k] = f16_pair_scaled(v[k], ex[m]);
                *(uint4*)(rA + 16u * (uint32_t)((bb * 8 + (qq & 7)) * 4 + (qq >> 3))) = make_uint4(hv[0], hv[1], hv[2], hv[3]);
                if constexpr (TYPE == T_Q8_0) {
                    float f[8];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        f[2 * k] = f16_to_f32(hv[k]);
                        f[2 * k + 1] = f16_to_f32(hv[k] >> 16);
                    }
                    float sm = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
                    sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
                    sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x4E, 0xF, 0xF, false));
                    if ((qq & 3) == 0) wS[8 * bb + (qq >> 2)] = sm;
                }
            }
        }
    };
#pragma unroll
    for (int i = 0; i < XI && i < kRing / 2; ++i) stage(i);
    // the ring slot of block b, and the restaging of blocks 2i, 2i + 1 (i >= 2) before group gi
    auto slot = [](int b) { return b & (kRing - 1); };
    auto restage = [&](int gi) {
#pragma unroll
        for (int i = kRing / 2; i < XI; ++i)
            if (gi == (2 * i) / G::GS) stage(i);
    };

    // 4. group loop: the lane's weights of a group, made into operands once, against every row.
    // The diagonal lane 16g + 4g + m reads row m's entries (the others stay zero).
    const int n = lane & 15, g = lane >> 4;
    const uint32_t aLane = lds_addr(wA) + (uint32_t)((n - 4 * g) & 3) * (uint32_t)AR::kBytes + 16u * (uint32_t)g;
    const uint64_t dmask = diag_mask(MR);
    const uint32_t rrow = (uint32_t)n * (uint32_t)(G::kPitch * G::GS);
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    u32x4_t A[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) A[t] = u32x4_t{0u, 0u, 0u, 0u};
    auto sums = [&](int m) { return (const float*)(wA + m * AR::kBytes + AR::kSumOff); };
    if constexpr (TYPE == T_Q4_K) {
        const HdrSel hs = hdr_sel(g);
        const CodeK ck = code_k();
        for (int gi = 0; gi < NG; ++gi) {
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            Raw R[G::GS];
#pragma unroll
            for (int bb = 0; bb < G::GS; ++bb) {
                const uint8_t* p = wW + rrow + G::kPitch * bb;
                R[bb].h = *(const uint4*)p;
                R[bb].q0 = *(const uint4*)(p + 16 + 32 * g);
                R[bb].q1 = *(const uint4*)(p + 32 + 32 * g);
            }
            if (gi + 1 < NG) {
                regs_consumed(R);   // the slice has been read: refill it
                const int nxt = (gi + 1) * G::GS;
                dma.issue(wr, wW, kb0 + nxt, bpk - nxt);
            }
            restage(gi);
#pragma unroll
            for (int bb = 0; bb < G::GS; ++bb) {
                const int b = slot(gi * G::GS + bb);
                a_reads(A, aLane + 512u * (uint32_t)b, dmask);
                float2 as[MR];
#pragma unroll
                for (int m = 0; m < MR; ++m) as[m] = *(const float2*)(sums(m) + (b * 4 + g) * 2);
                q4k_block_rows<MR>(R[bb], A, as, hs, ck, acc);
            }
        }
    } else if constexpr (TYPE == T_Q6_K || TYPE == T_Q8_0) {
        typedef typename std::conditional<TYPE == T_Q6_K, RawQ6, RawQ8>::type RawT;
        for (int gi = 0; gi < NG; ++gi) {
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            RawT R[G::GS];
#pragma unroll
            for (int bb = 0; bb < G::GS; ++bb) {
                if constexpr (TYPE == T_Q6_K)
                    R[bb] = q6_read(wW + rrow + G::kPitch * bb, g);
                else
                    R[bb] = q8_read(wW + rrow + G::kPitch * bb, g);
            }
            if (gi + 1 < NG) {
                regs_consumed(R);   // the slice has been read: refill it
                const int nxt = (gi + 1) * G::GS;
                dma.issue(wr, wW, kb0 + nxt, bpk - nxt);
            }
            restage(gi);
#pragma unroll
            for (int bb = 0; bb < G::GS; ++bb) {
                const int b = slot(gi * G::GS + bb);
                a_reads(A, aLane + 512u * (uint32_t)b, dmask);
                if constexpr (TYPE == T_Q6_K) {
                    float4 sg[MR];
#pragma unroll
                    for (int m = 0; m < MR; ++m) sg[m] = *(const float4*)(sums(m) + 16 * b + 4 * g);
                    q6_block_rows<MR>(R[bb], A, sg, g, acc);
                } else {
                    float2 s32[MR];
#pragma unroll
                    for (int m = 0; m < MR; ++m) s32[m] = *(const float2*)(sums(m) + 8 * b + 2 * g);
                    q8_block_rows<MR>(R[bb], A, s32, acc);
                }
            }
        }
    } else {
        // 16 rows x 1 block: two chains (MFMAs 0..3 and 4..7 of every block) over the whole part
        f32x4_t D0 = {0.f, 0.f, 0.f, 0.f}, D1 = {0.f, 0.f, 0.f, 0.f};
        for (int gi = 0; gi < NG; ++gi) {
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            const uint8_t* p = wW + rrow + 128 * g;
            Raw128 R[1];
#pragma unroll
            for (int s = 0; s < 8; ++s) R[0].v[s] = *(const uint4*)(p + 16 * s);
            if (gi + 1 < NG) {
                regs_consumed(R);   // the slice has been read: refill it
                dma.issue(wr, wW, kb0 + gi + 1, bpk - gi - 1);
            }
            restage(gi);
            a_reads(A, aLane + 512u * (uint32_t)slot(gi), dmask);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const u32x4_t b0 = {R[0].v[s].x, R[0].v[s].y, R[0].v[s].z, R[0].v[s].w};
                const u32x4_t b1 = {R[0].v[4 + s].x, R[0].v[4 + s].y, R[0].v[4 + s].z, R[0].v[4 + s].w};
                if constexpr (TYPE == T_F16) {
                    D0 = mfma_h(A[s], b0, D0);
                    D1 = mfma_h(A[4 + s], b1, D1);
                } else {
                    D0 = mfma(A[s], b0, D0);
                    D1 = mfma(A[4 + s], b1, D1);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = D0[m] + D1[m];
    }
    // a wave with no blocks still has its (all-zero) first group in flight
    __builtin_amdgcn_s_waitcnt(kWaitVm0);

    // 5. per row: reduce over the four K-groups (scaled back for fp16 operands), then across the
    // four parts in order
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float a = acc[m];
        a += __shfl_xor(a, 16, 64);
        a += __shfl_xor(a, 32, 64);
        if constexpr (kHalf) a = __builtin_ldexpf(a, ex[m]);
        if (lane < kTR) red[(m * kMixW + w) * kTR + lane] = a;
    }
    __syncthreads();
    const int m = tid / kTR, rr = tid - m * kTR;
    if (m < MR && m < M && rr < nvalid) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < kMixW; ++k) v += red[(m * kMixW + k) * kTR + rr];
        const int64_t row = T.row0 + r0 + rr;
        Y[(int64_t)m * ys + row] = (uint16_t)bf16_rne(v);
        if (Yf) Yf[(int64_t)m * ys + row] = v;
    }
}

template <int XI, int MR>
__global__ __launch_bounds__(kMixW * 64) void k_mixed(MixArgs args, const uint16_t* __restrict__ X, int K, int M,
                                                      uint16_t* __restrict__ Y, float* __restrict__ Yf, int64_t ys) {
    typedef ActRegion AR;
    // the staged activations live in a static LDS object of their own and the weight
    // slices in the dynamic one, so the compiler can tell the staging writes from the
    // direct-to-LDS loads in flight and does not make them wait for those
    __shared__ __align__(16) uint8_t s_act[kMixW * MR * AR::kBytes];
    __shared__ float red[MR * kMixW * kTR];
    extern __shared__ __align__(16) uint8_t s_w[];
    const int bid = blockIdx.x;
    const int wg = bid < args.split ? bid : args.nwg - 1 - (bid - args.split);
    int t = 0;
    while (t + 1 < args.n && args.t[t + 1].wg0 <= wg) ++t;
    const MixTile T = args.t[t];
    const int grp = wg - T.wg0;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t* wA = s_act + w * MR * AR::kBytes;
    uint8_t* wW = s_w + w * kSliceBytes;
    switch (T.type) {
        case T_Q4_K: mix_body<T_Q4_K, XI, MR>(T, grp, X, K, M, wA, wW, red, Y, Yf, ys); break;
        case T_Q6_K: mix_body<T_Q6_K, XI, MR>(T, grp, X, K, M, wA, wW, red, Y, Yf, ys); break;
        case T_Q8_0: mix_body<T_Q8_0, XI, MR>(T, grp, X, K, M, wA, wW, red, Y, Yf, ys); break;
        case T_F16: mix_body<T_F16, XI, MR>(T, grp, X, K, M, wA, wW, red, Y, Yf, ys); break;
        default: mix_body<T_BF16, XI, MR>(T, grp, X, K, M, wA, wW, red, Y, Yf, ys); break;
    }
}

// Blocks per wave that k_mixed<XI> loads as XI 16-B pieces per lane and row (every type's groups
// rounded up to whole groups must fit): 2 XI blocks.  A wave's bpk blocks round up to
// max(3 ceil(bpk / 3), 2 ceil(bpk / 2)) = 3, 3, 4, 6, 6, 6, 9, 9, ... blocks, so 1-3 blocks per
// wave take XI = 2, 4-6 take XI = 3 and 7-16 take XI = 8.
int mix_xi(int64_t K) {
    const int nsb = (int)(K / QK_K);
    const int bpk = (nsb + kMixW - 1) / kMixW;
    const int need = (bpk + 2) / 3 * 3 > (bpk + 1) / 2 * 2 ? (bpk + 2) / 3 * 3 : (bpk + 1) / 2 * 2;
    return need <= 4 ? 2 : need <= 6 ? 3 : need <= 16 ? 8 : 0;
}

// Activation rows per launch: four up to 6 blocks per wave (K <= 6144); beyond (K <= 16384) the
// rows' eight piece registers per lane leave room for two.
int mix_rows(int xi) { return xi <= 3 ? 4 : 2; }

bool mix_type(int t) { return t == T_Q4_K || t == T_Q6_K || t == T_Q8_0 || t == T_F16 || t == T_BF16; }

}  // namespace

bool gemv_mixed_supported(int type, int64_t K) {
    return mix_type(type) && K >= QK_K && K % QK_K == 0 && mix_xi(K) != 0;
}

// One launch over all tiles per pass of up to mix_rows(XI) activation rows; row m of the
// output starts at y + m * ys.  Rows of y outside the tiles are untouched.
// Workgroup order.  The 16-row groups differ up to 3.6x in bytes (Q4_K 144 B per 256 weights,
// F16 512 B).  The groups are ordered by their tile's bytes per row, heaviest first; the first
// workgroup per CU takes them in that order and the workgroups beyond take them from the
// lightest end, so a CU that runs two at once pairs a heavy group with a light one, and a CU
// that gets a later workgroup once it has finished one takes a light one.  Results do not
// depend on the order.
hipError_t launch_gemv_mixed(const aipu_tile_desc* tiles, int n_tiles, int64_t K, const uint16_t* x, int64_t M,
                             uint16_t* y, float* y_f32, int64_t ys, hipStream_t st) {
    if (n_tiles < 1 || n_tiles > AIPU_MAX_TILES || M < 1) return hipErrorInvalidValue;
    int order[AIPU_MAX_TILES];
    for (int i = 0; i < n_tiles; ++i) {
        const aipu_tile_desc& d = tiles[i];
        if (!gemv_mixed_supported(d.ggml_type, K) || d.nrows < 1 || d.nrows > (1LL << 30)) return hipErrorInvalidValue;
        int j = i;   // stable insertion by bytes per 256 weights, descending
        while (j > 0 && type_bytes(tiles[order[j - 1]].ggml_type) * 256 / type_qk(tiles[order[j - 1]].ggml_type) <
                            type_bytes(d.ggml_type) * 256 / type_qk(d.ggml_type)) {
            order[j] = order[j - 1];
            --j;
        }
        order[j] = i;
    }
    MixArgs a{};
    int64_t nwg = 0;
    for (int i = 0; i < n_tiles; ++i) {
        const aipu_tile_desc& d = tiles[order[i]];
        a.t[i] = MixTile{(const uint8_t*)d.w, d.row0, (int32_t)d.nrows, d.ggml_type, (int32_t)nwg, 0};
        nwg += (d.nrows + kTR - 1) / kTR;
        if (nwg > (1LL << 30)) return hipErrorInvalidValue;
    }
    a.nwg = (int)nwg;
    a.split = (int)(nwg < device_cu_count() ? nwg : device_cu_count());
    a.n = n_tiles;
    const dim3 grid((unsigned)nwg), block(kMixW * 64);
    const size_t lds = (size_t)kMixW * kSliceBytes;
    const int xi = mix_xi(K), mrmax = mix_rows(xi);
    for (int64_t m0 = 0; m0 < M;) {
        const int rows = (int)(M - m0 < mrmax ? M - m0 : mrmax);
        const uint16_t* xm = x + m0 * K;
        uint16_t* ym = y + m0 * ys;
        float* yfm = y_f32 ? y_f32 + m0 * ys : nullptr;
        const int mr = rows > 2 ? 4 : rows;
#define AIPU_MIX(XV, MV) \
    if (xi == XV && mr == MV) hipLaunchKernelGGL((k_mixed<XV, MV>), grid, block, lds, st, a, xm, (int)K, rows, ym, yfm, ys);
        AIPU_MIX(2, 1) AIPU_MIX(2, 2) AIPU_MIX(2, 4)
        AIPU_MIX(3, 1) AIPU_MIX(3, 2) AIPU_MIX(3, 4)
        AIPU_MIX(8, 1) AIPU_MIX(8, 2)
#undef AIPU_MIX
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        m0 += rows;
    }
    return hipSuccess;
}

}  // namespace aipu
