// Mixed-type GEMV (tolerance mode, MR <= 4 activation rows per launch): one launch over a list of tiles,
// each a run of output rows stored as Q4_K, Q6_K, Q8_0, F16 or BF16 -- the per-column
// w_type mux of src/glm_matmul_q4k.v:76-101,197-259 over the tile sequence of
// tools/q4k_mixed_gen.py:382-440.  A single-tile call serves the plain GEMV of the types
// other than Q4_K.
//
// Workgroup.  Four waves own one 16-row group of one tile (8 rows for F16 / BF16); wave w
// takes the w-th quarter of the row's 256-weight blocks.  Each wave stages its own activations, then streams its 16
// rows group by group (GS blocks per group) into its own LDS slice with direct-to-LDS buffer
// loads (16 consecutive bytes per lane, so one instruction covers ~1 KB of row bytes), and
// copies a group into registers before the next group's loads are issued into the slice.
// The four parts are added in fixed order, so results are deterministic.  With MR rows each
// wave stages every row's activations and applies each group of weights, decoded once in
// registers, to all of them: the weights are read once per launch, and each row's sums are
// formed exactly as in a one-row launch (the rows of a batch equal their single-row results).
//
// Lane layout: lane 16g + n works on row n of the group and on weights 64g..64g+63 of every
// block (a Q6_K lane instead takes half g>>1, positions l = 16(g&1)..+15 of the four
// 32-position runs, which are the same 64 weights in the order the Q6_K bytes store them).
// F16 / BF16 groups are 8 rows x 2 blocks (the same 8 KB as 16 rows x 1 block, in half the
// groups, so a wave waits for half as many copies): lane 16g + n takes row n & 7 and block
// n >> 3 of the group.  (Q6_K and Q8_0 groups of 8 rows x 4 blocks, two blocks per lane,
// measured slower: their decode is VALU-bound.)
//
// Arithmetic.  Q4_K runs on the matrix cores (mfma_gemv.hpp).  The other types decode in
// VALU registers against fp32 activations staged in LDS, with partial sums per scale group
// (fp32 FMA), then one scaled add per group:
//   Q6_K (tools/q4k_ref.py:105-124): sum_k a_k w_k = f32(d*sc) * (sum a_k c_k - 32 sum a_k),
//        c_k = 6-bit code, per 16-weight scale group;
//   Q8_0 (tools/q4k_ref.py:126-129): d * (sum a_k (q_k + 128) - 128 sum a_k), the biased code
//        q + 128 = (byte ^ 0x80) converted with one v_cvt_f32_ubyte;
//   F16 / BF16 (tools/glm_model_q4k_ref.py:61-63): exact conversion, FMA.
// The order of additions differs from the reference's sequential MAC, so this is the
// tolerance path; the reference-order kernel (gemv_ref.hip) is the bit-exact one.
#include "common.hpp"
#include "launch.hpp"
#include "mfma_gemv.hpp"

namespace aipu {

using namespace mg;

namespace {

constexpr int kMixW = 4;                  // waves per workgroup (= K parts)
constexpr int kSliceBytes = 9 * 1024;     // per-wave weight slice: the largest group below

// Bytes of one 256-weight block of one row in memory (kBlk) and in the LDS slice (kPitch),
// and blocks per streamed group (GS).  A Q6_K block is copied as 14 whole 16-B pieces (224
// bytes of LDS) so that every block starts 16-B aligned: pieces 0..12 are bytes 0..207 and
// piece 13 is bytes 194..209, so no piece reaches past the block (d lands at LDS byte 222).
// Q8_0 "blocks" are runs of eight 34-B ggml blocks.
template <int TYPE>
struct Geom;
template <>
struct Geom<T_Q4_K> {
    static constexpr int kBlk = 144, kPitch = 144, GS = 3, kRows = kTR;
};
template <>
struct Geom<T_Q6_K> {
    static constexpr int kBlk = 210, kPitch = 224, GS = 2, kRows = kTR;
};
template <>
struct Geom<T_Q8_0> {
    static constexpr int kBlk = 272, kPitch = 272, GS = 2, kRows = kTR;
};
template <>
struct Geom<T_F16> {
    static constexpr int kBlk = 512, kPitch = 512, GS = 2, kRows = kTR / 2;
};
template <>
struct Geom<T_BF16> {
    static constexpr int kBlk = 512, kPitch = 512, GS = 2, kRows = kTR / 2;
};
// Output rows per workgroup of a tile of type t.
int mix_tile_rows(int t) { return t == T_F16 || t == T_BF16 ? kTR / 2 : kTR; }

// Direct-to-LDS copy of one group: piece j (16 B) of the slice is piece p of block b of row
// r, j = (r * GS + b) * kPitch / 16 + p.  Lanes past the last piece, and blocks past the
// wave's range, read through the out-of-range offset (zeros, no memory access).
template <int TYPE>
struct MixDma {
    typedef Geom<TYPE> G;
    static constexpr int kP16 = G::kPitch / 16;
    static constexpr int kRowPieces = G::GS * kP16;
    static constexpr int kPieces = G::kRows * kRowPieces;
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

// -------------------------------------------------------------- per-type blocks
// Q6_K: the lane's bytes of one block (ql runs at 64h + o and 64h + 32 + o, qh at
// 128 + 32h + o, the 8 scales of half h, d).
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

__device__ __forceinline__ float ubyte(uint32_t v, int j) { return (float)((v >> (8 * j)) & 0xFFu); }

// 16 fp32 FMAs of four code dwords against 16 consecutive activations.
__device__ __forceinline__ float dot16(const uint32_t (&c)[4], const float* a) {
    const float4 a0 = *(const float4*)(a), a1 = *(const float4*)(a + 4);
    const float4 a2 = *(const float4*)(a + 8), a3 = *(const float4*)(a + 12);
    float s0 = ubyte(c[0], 0) * a0.x, s1 = ubyte(c[0], 1) * a0.y;
    s0 = __builtin_fmaf(ubyte(c[0], 2), a0.z, s0);
    s1 = __builtin_fmaf(ubyte(c[0], 3), a0.w, s1);
    s0 = __builtin_fmaf(ubyte(c[1], 0), a1.x, s0);
    s1 = __builtin_fmaf(ubyte(c[1], 1), a1.y, s1);
    s0 = __builtin_fmaf(ubyte(c[1], 2), a1.z, s0);
    s1 = __builtin_fmaf(ubyte(c[1], 3), a1.w, s1);
    s0 = __builtin_fmaf(ubyte(c[2], 0), a2.x, s0);
    s1 = __builtin_fmaf(ubyte(c[2], 1), a2.y, s1);
    s0 = __builtin_fmaf(ubyte(c[2], 2), a2.z, s0);
    s1 = __builtin_fmaf(ubyte(c[2], 3), a2.w, s1);
    s0 = __builtin_fmaf(ubyte(c[3], 0), a3.x, s0);
    s1 = __builtin_fmaf(ubyte(c[3], 1), a3.y, s1);
    s0 = __builtin_fmaf(ubyte(c[3], 2), a3.z, s0);
    s1 = __builtin_fmaf(ubyte(c[3], 3), a3.w, s1);
    return s0 + s1;
}

// One Q6_K block on lane 16g + n.  act: the block's 256 fp32 activations; s16: its 16
// sums of 16.  Position 128h + 32t + l takes the low (t < 2) or high nibble of
// ql[64h + 32(t&1) + l] and bits 2t..2t+1 of qh[32h + l]; scale index = position >> 4.
__device__ __forceinline__ float q6_block(const RawQ6& r, const float* act, const float* s16, int g, float acc) {
    const int h = g >> 1, hi = g & 1, o = 16 * hi;
    const float d = f16_to_f32(r.d);
    const uint32_t ql0[4] = {r.ql0.x, r.ql0.y, r.ql0.z, r.ql0.w};
    const uint32_t ql1[4] = {r.ql1.x, r.ql1.y, r.ql1.z, r.ql1.w};
    const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        uint32_t c[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t ql = t & 1 ? ql1[k] : ql0[k];
            const uint32_t nib = (t < 2 ? ql : ql >> 4) & 0x0F0F0F0Fu;
            const uint32_t hb = t == 0 ? qh[k] << 4 : t == 1 ? qh[k] << 2 : t == 2 ? qh[k] : qh[k] >> 2;
            c[k] = nib | (hb & 0x30303030u);
        }
        const float s = dot16(c, act + 128 * h + 32 * t + o);
        const float sg = s16[8 * h + 2 * t + hi];
        const int sci = hi + 2 * t;   // byte of the half's 8 scales
        const uint32_t scw = sci < 4 ? r.sc.x : r.sc.y;
        const int sc = (int)(int8_t)(uint8_t)(scw >> (8 * (sci & 3)));
        const float dsc = d * (float)sc;
        acc = __builtin_fmaf(dsc, __builtin_fmaf(-32.0f, sg, s), acc);
    }
    return acc;
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

__device__ __forceinline__ float q8_block(const RawQ8& r, const float* act, const float* s16, int g, float acc) {
    uint32_t x[17];
#pragma unroll
    for (int k = 0; k < 17; ++k) x[k] = r.w[k] ^ 0x80808080u;   // bytes -> q + 128
    const float* a = act + 64 * g;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int b0 = half ? 36 : 2;   // byte offset of the 32 codes
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i += 2) {
            s0 = __builtin_fmaf(ubyte(x[(b0 + i) >> 2], (b0 + i) & 3), a[32 * half + i], s0);
            s1 = __builtin_fmaf(ubyte(x[(b0 + i + 1) >> 2], (b0 + i + 1) & 3), a[32 * half + i + 1], s1);
        }
        const float d = f16_to_f32(half ? r.w[8] >> 16 : r.w[0]);
        const float sg = s16[4 * g + 2 * half] + s16[4 * g + 2 * half + 1];
        acc = __builtin_fmaf(d, __builtin_fmaf(-128.0f, sg, s0 + s1), acc);
    }
    return acc;
}

// F16 / BF16: the lane's 64 weights (128 B).
struct Raw128 {
    uint4 v[8];
};

template <int TYPE>
__device__ __forceinline__ float f16_block(const Raw128& r, const float* act, int g, float acc) {
    const float* a = act + 64 * g;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t w[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
        const float4 a0 = *(const float4*)(a + 8 * i), a1 = *(const float4*)(a + 8 * i + 4);
        const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float lo, hi;
            if constexpr (TYPE == T_F16) {
                lo = f16_to_f32(w[k]);
                hi = f16_to_f32(w[k] >> 16);
            } else {
                lo = __uint_as_float(w[k] << 16);
                hi = __uint_as_float(w[k] & 0xFFFF0000u);
            }
            s0 = __builtin_fmaf(lo, av[2 * k], s0);
            s1 = __builtin_fmaf(hi, av[2 * k + 1], s1);
        }
    }
    return acc + (s0 + s1);
}

// ------------------------------------------------------------------ kernel
struct MixTile {
    const uint8_t* w;
    int64_t row0;
    int32_t nrows, type;
    int32_t wg0, pad;   // first workgroup of the tile
};

struct MixArgs {
    MixTile t[AIPU_MAX_TILES];
    int n;
};

// Per-wave activation region: fp32 activations [2XI blocks][256] then 16-weight sums
// [2XI][16] (VALU types), or the Q4_K operand layout [2XI][512 B] then its 32-weight sums.
template <int XI>
struct ActRegion {
    static constexpr int kBlocks = 2 * XI;
    static constexpr int kBytes = kBlocks * (1024 + 64);
    static constexpr int kSumOffF = kBlocks * 1024;   // VALU: sums16
    static constexpr int kSumOffQ = kBlocks * 512;    // Q4_K: sums32
};

template <int TYPE, int XI, int MR>
__device__ __forceinline__ void mix_body(const MixTile& T, int grp, const uint16_t* __restrict__ X, int K, int M,
                                         uint8_t* wA, uint8_t* wW, float* red, uint16_t* Y, float* Yf, int64_t ys) {
    typedef Geom<TYPE> G;
    typedef ActRegion<XI> AR;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nsb = K / QK_K;
    const int kb0 = w * nsb / kMixW, kb1 = (w + 1) * nsb / kMixW;
    const int bpk = kb1 - kb0;
    const int NG = (bpk + G::GS - 1) / G::GS;
    const int64_t rb = (int64_t)nsb * G::kBlk;
    const int r0 = grp * G::kRows;
    const int nvalid = T.nrows - r0 < G::kRows ? T.nrows - r0 : G::kRows;

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

    // 3. stage (every piece of the region, so blocks past bpk hold zeros); row m at m * kBytes
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        uint8_t* rA = wA + m * AR::kBytes;
        if constexpr (TYPE == T_Q4_K) {
            float* wS = (float*)(rA + AR::kSumOffQ);
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const int q = lane + 64 * i;
                const uint32_t ones = 0x3F803F80u;
                float sm = 0.f;
                sm = dot2(xv[m][i].x, ones, sm);
                sm = dot2(xv[m][i].y, ones, sm);
                sm = dot2(xv[m][i].z, ones, sm);
                sm = dot2(xv[m][i].w, ones, sm);
                sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
                sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0x4E, 0xF, 0xF, false));
                const int bb = q >> 5, gg = (q >> 3) & 3, t = q & 7;
                *(u32x4_t*)(rA + 16u * (uint32_t)((bb * 8 + t) * 4 + gg)) = act_perm(xv[m][i]);
                if ((q & 3) == 0) wS[(bb * 4 + gg) * 2 + ((q >> 2) & 1)] = sm;
            }
        } else {
            float* wF = (float*)rA;
            float* wS = (float*)(rA + AR::kSumOffF);
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const int q = lane + 64 * i;
                const uint32_t v[4] = {xv[m][i].x, xv[m][i].y, xv[m][i].z, xv[m][i].w};
                float f[8];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    f[2 * k] = __uint_as_float(v[k] << 16);
                    f[2 * k + 1] = __uint_as_float(v[k] & 0xFFFF0000u);
                }
                float sm = ((f[0] + f[1]) + (f[2] + f[3])) + ((f[4] + f[5]) + (f[6] + f[7]));
                sm += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sm), 0xB1, 0xF, 0xF, false));
                *(float4*)(wF + 8 * q) = make_float4(f[0], f[1], f[2], f[3]);
                *(float4*)(wF + 8 * q + 4) = make_float4(f[4], f[5], f[6], f[7]);
                if ((q & 1) == 0) wS[q >> 1] = sm;
            }
        }
    }

    // 4. group loop: the lane's weights of a group, decoded once, against every row
    const int n = lane & 15, g = lane >> 4;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = 0.f;
    if constexpr (TYPE == T_Q4_K) {
        u32x4_t A[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) A[t] = u32x4_t{0u, 0u, 0u, 0u};
        const HdrSel hs = hdr_sel(g);
        const CodeK ck = code_k();
        f32x4_t dlo = {0.f, 0.f, 0.f, 0.f}, dhi = {0.f, 0.f, 0.f, 0.f};
        const uint32_t rrow = (uint32_t)n * (uint32_t)(G::kPitch * G::GS);
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
#pragma unroll
            for (int bb = 0; bb < G::GS; ++bb) {
                const int b = gi * G::GS + bb;
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const uint8_t* rA = wA + m * AR::kBytes;
                    a_reads(A, lds_addr(rA + 512u * (uint32_t)b + 16u * (uint32_t)g), diag_mask(1));
                    const float2 as = *(const float2*)((const float*)(rA + AR::kSumOffQ) + (b * 4 + g) * 2);
                    acc[m] = q4k_block1(R[bb], A, as, hs, ck, dlo, dhi, acc[m]);
                }
            }
        }
    } else {
        const uint32_t rrow = (uint32_t)n * (uint32_t)(G::kPitch * G::GS);
        for (int gi = 0; gi < NG; ++gi) {
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            const uint8_t* p = wW + rrow;
            if constexpr (TYPE == T_Q6_K) {
                RawQ6 R[G::GS];
#pragma unroll
                for (int bb = 0; bb < G::GS; ++bb) R[bb] = q6_read(p + G::kPitch * bb, g);
                if (gi + 1 < NG) {
                    regs_consumed(R);   // the slice has been read: refill it
                    const int nxt = (gi + 1) * G::GS;
                    dma.issue(wr, wW, kb0 + nxt, bpk - nxt);
                }
#pragma unroll
                for (int bb = 0; bb < G::GS; ++bb) {
                    const int b = gi * G::GS + bb;
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        const uint8_t* rA = wA + m * AR::kBytes;
                        acc[m] = q6_block(R[bb], (const float*)rA + 256 * b, (const float*)(rA + AR::kSumOffF) + 16 * b, g, acc[m]);
                    }
                }
            } else if constexpr (TYPE == T_Q8_0) {
                RawQ8 R[G::GS];
#pragma unroll
                for (int bb = 0; bb < G::GS; ++bb) R[bb] = q8_read(p + G::kPitch * bb, g);
                if (gi + 1 < NG) {
                    regs_consumed(R);   // the slice has been read: refill it
                    const int nxt = (gi + 1) * G::GS;
                    dma.issue(wr, wW, kb0 + nxt, bpk - nxt);
                }
#pragma unroll
                for (int bb = 0; bb < G::GS; ++bb) {
                    const int b = gi * G::GS + bb;
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        const uint8_t* rA = wA + m * AR::kBytes;
                        acc[m] = q8_block(R[bb], (const float*)rA + 256 * b, (const float*)(rA + AR::kSumOffF) + 16 * b, g, acc[m]);
                    }
                }
            } else {
                // 8 rows x 2 blocks: this lane's row n & 7, block n >> 3 of the group (a block
                // past the wave's range reads zeros, against zero-staged activations)
                const int bb = n >> 3;
                const uint8_t* q = wW + (uint32_t)(n & 7) * (uint32_t)(G::kPitch * G::GS) + G::kPitch * bb + 128 * g;
                Raw128 R[1];
#pragma unroll
                for (int i = 0; i < 8; ++i) R[0].v[i] = *(const uint4*)(q + 16 * i);
                if (gi + 1 < NG) {
                    regs_consumed(R);   // the slice has been read: refill it
                    const int nxt = (gi + 1) * G::GS;
                    dma.issue(wr, wW, kb0 + nxt, bpk - nxt);
                }
                const int b = gi * G::GS + bb;
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    acc[m] = f16_block<TYPE>(R[0], (const float*)(wA + m * AR::kBytes) + 256 * b, g, acc[m]);
            }
        }
    }
    // a wave with no blocks still has its (all-zero) first group in flight
    __builtin_amdgcn_s_waitcnt(kWaitVm0);

    // 5. per row: reduce over the four K-groups (and an 8-row group's two blocks), then
    // across the four parts in order
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float a = acc[m];
        a += __shfl_xor(a, 16, 64);
        a += __shfl_xor(a, 32, 64);
        if constexpr (G::kRows < kTR) a += __shfl_xor(a, 8, 64);
        if (lane < G::kRows) red[(m * kMixW + w) * kTR + lane] = a;
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
    typedef ActRegion<XI> AR;
    // the staged activations live in a static LDS object of their own and the weight
    // slices in the dynamic one, so the compiler can tell the staging writes from the
    // direct-to-LDS loads in flight and does not make them wait for those
    __shared__ __align__(16) uint8_t s_act[kMixW * MR * AR::kBytes];
    __shared__ float red[MR * kMixW * kTR];
    extern __shared__ __align__(16) uint8_t s_w[];
    const int wg = blockIdx.x;
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

// Blocks per wave the activation region of k_mixed<XI> holds (every type's groups rounded
// up to whole groups must fit): 2 XI blocks.  A wave's bpk blocks round up to
// max(3 ceil(bpk / 3), 2 ceil(bpk / 2)) = 3, 3, 4, 6, 6, 6, 9, 9, ... blocks, so 1-3 blocks per
// wave take XI = 2, 4-6 take XI = 3 and 7-16 take XI = 8.
int mix_xi(int64_t K) {
    const int nsb = (int)(K / QK_K);
    const int bpk = (nsb + kMixW - 1) / kMixW;
    const int need = (bpk + 2) / 3 * 3 > (bpk + 1) / 2 * 2 ? (bpk + 2) / 3 * 3 : (bpk + 1) / 2 * 2;
    return need <= 4 ? 2 : need <= 6 ? 3 : need <= 16 ? 8 : 0;
}

// Activation rows per launch that the LDS holds beside the weight slices (160 KB): four up
// to 6 blocks per wave (K <= 6144), one beyond (K <= 16384).
int mix_rows(int xi) { return xi <= 3 ? 4 : 1; }

bool mix_type(int t) { return t == T_Q4_K || t == T_Q6_K || t == T_Q8_0 || t == T_F16 || t == T_BF16; }

}  // namespace

bool gemv_mixed_supported(int type, int64_t K) {
    return mix_type(type) && K >= QK_K && K % QK_K == 0 && mix_xi(K) != 0;
}

// One launch over all tiles per pass of up to mix_rows(XI) activation rows; row m of the
// output starts at y + m * ys.  Rows of y outside the tiles are untouched.
hipError_t launch_gemv_mixed(const aipu_tile_desc* tiles, int n_tiles, int64_t K, const uint16_t* x, int64_t M,
                             uint16_t* y, float* y_f32, int64_t ys, hipStream_t st) {
    if (n_tiles < 1 || n_tiles > AIPU_MAX_TILES || M < 1) return hipErrorInvalidValue;
    MixArgs a{};
    int64_t nwg = 0;
    for (int i = 0; i < n_tiles; ++i) {
        const aipu_tile_desc& d = tiles[i];
        if (!gemv_mixed_supported(d.ggml_type, K) || d.nrows < 1 || d.nrows > (1LL << 30)) return hipErrorInvalidValue;
        a.t[i] = MixTile{(const uint8_t*)d.w, d.row0, (int32_t)d.nrows, d.ggml_type, (int32_t)nwg, 0};
        nwg += (d.nrows + mix_tile_rows(d.ggml_type) - 1) / mix_tile_rows(d.ggml_type);
        if (nwg > (1LL << 30)) return hipErrorInvalidValue;
    }
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
        AIPU_MIX(8, 1)
#undef AIPU_MIX
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        m0 += rows;
    }
    return hipSuccess;
}

}  // namespace aipu
