// Prefill GEMM for large M on the matrix cores (tolerance mode):
//     y[M][N] = bf16(x[M][K] . dequant(W)^T),   W = Q4_K row blocks [N][K/256].
// No reference counterpart beyond M independent matmul_q4k_col rows (tools/q4k_ref.py:86-92).
//
// Arithmetic.  For activation row m, weight row n and super-block b (256 weights),
//     sum_k a_k w_k = d * sum_k a_k (sc_s(k) * q_k)  -  dmin * sum_s m_s * (sum_{k in s} a_k),
// the factorised form of w = d*sc*q - dmin*m (tools/q4k_ref.py:53-59).
//   * sc*q is an integer in 0..945, exact in fp16, so the first sum runs on
//     v_mfma_f32_16x16x32_f16 with exact products and fp32 accumulation.
//   * Activations enter as fp16 after scaling row m by 2^-e_m, which puts the row's largest
//     magnitude in [2^14, 2^15): every bf16 value down to 2^-31 of the row maximum converts
//     exactly, smaller ones lose at most 2^-25 * 2^e_m.  The output is scaled back by 2^e_m.
//   * The min term runs on v_mfma_f32_16x16x32_bf16: the 8 sub-block sums of the (scaled,
//     fp16-rounded) activations, each split exactly into three bf16 terms hi + mid + lo,
//     against the 6-bit mins (exact in bf16).
//   * Per super-block: acc += d * D1 - dmin * D2 (two fp32 FMAs per output).
//
// Pre-pass (k_prefill_rowexp, k_prefill_pack) writes the scaled activations into a caller
// workspace in the order the GEMM reads them: for each 128-row tile and super-block one
// 72 KB chunk, [t][i][lane] 16-B MFMA operands (t = MFMA 0..7, i = 16-row subtile 0..7)
// then [i][lane] 16-B sum operands, so the GEMM stages a chunk into LDS with straight
// direct-to-LDS copies and every operand read is one conflict-free 1 KB ds_read_b128 sweep.
//
// K order inside a super-block.  Lane l = 16g + n of an MFMA supplies 8 K-values.  For the
// weights, lane group g reads qs piece g (bytes 16g..16g+15) and piece g+4 (64+16g..) of
// its row's block; MFMA t uses dword t%4 of piece (t<4 ? g : g+4).  A dword holds bytes
// j..j+3 of qs chunk c (32 bytes: low nibbles = sub-block 2c, high nibbles = 2c+1); its 8
// codes are taken as the fp16 pairs (b0,b2) (b1,b3) low, then (b0,b2) (b1,b3) high, so
//     K(t, g, e) = 64c + 32*(e >= 4) + 16*(g & 1) + 4*(t & 3) + {0, 2, 1, 3}[e & 3],
//     c = (t < 4 ? 0 : 2) + (g >> 1),
// and the pack kernel writes the activations in that order.  The sum operand of lane
// group g carries sub-blocks g and 4 + g: elements (hi, mid, lo, 0) of each.
//
// Code -> operand.  (v & 0x000F000F) | 0x64006400 is the fp16 pair 1024 + q, and one
// v_pk_fma_f16 with (sc, sc) and (-1024 sc, -1024 sc) leaves sc*q exactly; for the high
// nibbles (v & 0x00F000F0) | 0x64006400 = 1024 + 16q goes with (sc/16) and -64 sc.
//
// Tiles.  Workgroup = 4 waves (one per SIMD, up to 512 registers each) over a 128 x 256
// (M x N) output tile; wave w owns weight rows 64w..64w+63 of it (4 subtiles of 16) and all
// 128 activation rows (8 subtiles): 32 accumulator tiles, plus 32 per-super-block tiles.
// The activation chunk of super-block b+1 is copied into the other LDS stage and the
// wave's weight blocks of b+1 are loaded into the other register set while b computes.
// Workgroups sharing a weight tile are consecutive on one XCD (its L2 serves the re-reads).
#include "common.hpp"
#include "launch.hpp"

namespace aipu {

namespace {

constexpr int kBM = 128;                         // activation rows per workgroup
constexpr int kBN = 256;                         // weight rows per workgroup
constexpr int kWaves = 4;
constexpr int kMS = kBM / 16;                    // 16-row activation subtiles per wave
constexpr int kNS = kBN / kWaves / 16;           // 16-row weight subtiles per wave
constexpr int kChunkA = 8 * kMS * 64 * 16;       // fp16 operands of one super-block
constexpr int kChunkS = kMS * 64 * 16;           // sum operands
constexpr int kChunk = kChunkA + kChunkS;        // 73728 B
constexpr int kDmaPerWave = kChunk / 1024 / kWaves;
static_assert(kChunk % (1024 * kWaves) == 0, "chunk must split into whole 1 KB copies per wave");

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t f16_scaled(uint32_t bf, int e) {
    const float f = __builtin_ldexpf(bf16_to_f32(bf & 0xFFFFu), -e);
    return (uint32_t)__half_as_ushort(__float2half_rn(f));
}

// fp32 v = hi + mid + lo exactly, each a bf16 (top, middle, bottom 8 significant bits).
__device__ __forceinline__ void split3(float v, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
    const uint32_t h = __float_as_uint(v) & 0xFFFF0000u;
    const float r1 = v - __uint_as_float(h);
    const uint32_t md = __float_as_uint(r1) & 0xFFFF0000u;
    const float r2 = r1 - __uint_as_float(md);
    hi = h >> 16;
    mid = md >> 16;
    lo = __float_as_uint(r2) >> 16;
}

// Row exponent e_m: the largest |x| of row m scaled by 2^-e_m lies in [2^14, 2^15).  Rows
// that are all zero, hold inf/nan, or lie past M get e = 0.  One wave per row.
__global__ __launch_bounds__(256) void k_prefill_rowexp(const uint16_t* __restrict__ X, int64_t K, int M, int Mpad,
                                                        int32_t* __restrict__ rexp) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= Mpad) return;
    uint32_t mx = 0;
    if (row < M) {
        const uint16_t* xr = X + (int64_t)row * K;
        for (int64_t k = (int64_t)lane * 8; k < K; k += 512) {
            const uint4 v = *(const uint4*)(xr + k);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                mx = max(mx, w[q] & 0x7FFFu);
                mx = max(mx, (w[q] >> 16) & 0x7FFFu);
            }
        }
    }
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, s, 64));
    if (lane == 0) {
        int e = 0;
        if (mx != 0 && mx < 0x7F80u) {
            int ex;
            (void)frexpf(bf16_to_f32(mx), &ex);   // max = f * 2^ex, f in [0.5, 1)
            e = ex - 15;
        }
        rexp[row] = e;
    }
}

// One workgroup per (super-block b, 128-row tile mt): writes chunk (mt, b).
__global__ __launch_bounds__(256) void k_prefill_pack(const uint16_t* __restrict__ X, int64_t K, int M,
                                                      const int32_t* __restrict__ rexp, uint8_t* __restrict__ ws,
                                                      int nsb) {
    const int b = blockIdx.x, mt = blockIdx.y;
    uint8_t* chunk = ws + ((int64_t)mt * nsb + b) * kChunk;
    for (int idx = threadIdx.x; idx < kChunkA / 16; idx += 256) {
        const int t = idx / (kMS * 64), i = (idx / 64) % kMS, lane = idx & 63;
        const int r = lane & 15, g = lane >> 4;
        const int m = mt * kBM + i * 16 + r;
        uint4 out = make_uint4(0, 0, 0, 0);
        if (m < M) {
            const int e = rexp[m];
            const int c = (t < 4 ? 0 : 2) + (g >> 1);
            const int64_t k0 = (int64_t)b * QK_K + 64 * c + 16 * (g & 1) + 4 * (t & 3);
            const uint2 lo = *(const uint2*)(X + (int64_t)m * K + k0);        // x[k0 .. k0+3]
            const uint2 hi = *(const uint2*)(X + (int64_t)m * K + k0 + 32);   // x[k0+32 .. k0+35]
            out.x = f16_scaled(lo.x, e) | f16_scaled(lo.y, e) << 16;              // (k0, k0+2)
            out.y = f16_scaled(lo.x >> 16, e) | f16_scaled(lo.y >> 16, e) << 16;  // (k0+1, k0+3)
            out.z = f16_scaled(hi.x, e) | f16_scaled(hi.y, e) << 16;
            out.w = f16_scaled(hi.x >> 16, e) | f16_scaled(hi.y >> 16, e) << 16;
        }
        *(uint4*)(chunk + (int64_t)idx * 16) = out;
    }
    for (int idx = threadIdx.x; idx < kChunkS / 16; idx += 256) {
        const int i = idx / 64, lane = idx & 63;
        const int r = lane & 15, g = lane >> 4;
        const int m = mt * kBM + i * 16 + r;
        uint32_t o[4] = {0, 0, 0, 0};
        if (m < M) {
            const int e = rexp[m];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const uint16_t* p = X + (int64_t)m * K + (int64_t)b * QK_K + 32 * (g + 4 * q);
                float s = 0.f;
                for (int k = 0; k < 32; ++k) s += __half2float(__ushort_as_half((unsigned short)f16_scaled(p[k], e)));
                uint32_t h, md, l;
                split3(s, h, md, l);
                o[2 * q] = h | md << 16;
                o[2 * q + 1] = l;
            }
        }
        *(uint4*)(chunk + kChunkA + (int64_t)idx * 16) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, 0);
}

// Copy bytes [lo, lo + 1024 * kWaves * n) of chunk (mt, b) into `dst`: 1 KB per instruction,
// wave w takes every kWaves-th KB.
template <int NPW>
__device__ __forceinline__ void dma_chunk(const uint8_t* ws, int64_t chunk_index, uint32_t lo, uint8_t* dst, int w,
                                          int lane) {
    const __amdgpu_buffer_rsrc_t r = buf_rsrc(ws + chunk_index * kChunk, (uint32_t)kChunk);
#pragma unroll
    for (int k = 0; k < NPW; ++k) {
        const uint32_t kb = (uint32_t)(k * kWaves + w) * 1024u;
        dma16(r, dst + kb, lo + kb + 16u * (uint32_t)lane);
    }
}

// The wave's 64 weight rows of super-block b into its LDS slice, laid out [q][j][n] by
// 16-B piece q of the block (0 = header, 1 + p = qs piece p), row 16j + n: a lane group
// reading one piece of 16 rows touches 256 contiguous bytes.
constexpr int kSliceB = 9 * kNS * 16 * 16;   // 9216 B per wave
__device__ __forceinline__ void dma_blocks(__amdgpu_buffer_rsrc_t wr, uint32_t rb, int b, uint8_t* slice, int lane) {
    const int j = lane >> 4, n = lane & 15;
    const uint32_t row_off = (uint32_t)(16 * j + n) * rb + (uint32_t)b * 144u;
#pragma unroll
    for (int q = 0; q < 9; ++q) dma16(wr, slice + q * 1024, row_off + 16u * (uint32_t)q);
}

__device__ __forceinline__ uint4 lds_u4(const uint8_t* p) { return *(const uint4*)p; }

__device__ __forceinline__ h2_t h2bits(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
__device__ __forceinline__ uint32_t bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// get_scale_min_k4 (tools/q4k_ref.py:27-37) for the sub-blocks lane group g uses:
// sc of 2c, 2c+1 for qs chunk c = half*2 + (g >> 1), and the mins m_g, m_{4+g}.
struct ChunkK {
    h2_t sl, cl, sh, ch;   // low nibbles: sc, -1024 sc; high nibbles: sc/16, -64 sc
};

__device__ __forceinline__ ChunkK chunk_consts(const uint4& h, int g, int half) {
    const int ja = 2 * (g >> 1);
    const uint32_t s0 = h.y, s2 = h.w;
    uint32_t lo, hi;
    if (half == 0) {
        lo = (s0 >> (8 * ja)) & 63u;
        hi = (s0 >> (8 * ja + 8)) & 63u;
    } else {
        lo = ((s2 >> (8 * ja)) & 0xFu) | (((s0 >> (8 * ja + 6)) & 3u) << 4);
        hi = ((s2 >> (8 * ja + 8)) & 0xFu) | (((s0 >> (8 * ja + 14)) & 3u) << 4);
    }
    ChunkK k;
    const _Float16 l = (_Float16)(float)lo;
    const _Float16 u = (_Float16)((float)hi * 0.0625f);
    const h2_t neg = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    k.sl = h2_t{l, l};
    k.cl = k.sl * neg;
    k.sh = h2_t{u, u};
    k.ch = k.sh * neg;
    return k;
}

// bf16 operand of the min term: (m_g x4, m_{4+g} x4); the 4th element of each group meets
// a zero activation-sum term.
__device__ __forceinline__ u32x4_t min_operand(const uint4& h, int g) {
    const uint32_t s1 = h.z, s2 = h.w;
    const uint32_t mg = (s1 >> (8 * g)) & 63u;
    const uint32_t m4g = ((s2 >> (8 * g + 4)) & 0xFu) | (((s1 >> (8 * g + 6)) & 3u) << 4);
    const uint32_t bl = __float_as_uint((float)mg) >> 16, bh = __float_as_uint((float)m4g) >> 16;
    const uint32_t pl = bl | bl << 16, ph = bh | bh << 16;
    return u32x4_t{pl, pl, ph, ph};
}

// (v & mask) | bias in one v_and_or_b32: gfx9 VOP3 takes no literal and one scalar operand,
// so the masks sit in SGPRs and the bias in a VGPR the caller keeps live.
struct CodeMask {
    uint32_t lo, hi;   // 0x000F000F, 0x00F000F0 (SGPR)
    uint32_t bias;     // 0x64006400 (VGPR): fp16 1024 in both halves
};

__device__ __forceinline__ CodeMask code_mask() {
    CodeMask c;
    c.lo = __builtin_amdgcn_readfirstlane(0x000F000Fu);
    c.hi = __builtin_amdgcn_readfirstlane(0x00F000F0u);
    c.bias = 0x64006400u;
    return c;
}

__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t bias) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(bias));
    return r;
}

// The 8 fp16 operands sc*q of one MFMA from qs dword x.
__device__ __forceinline__ h8_t b_operand(uint32_t x, const ChunkK& k, const CodeMask& cm) {
    const uint32_t y = x >> 8;
    const h2_t p0 = __builtin_elementwise_fma(h2bits(and_or(x, cm.lo, cm.bias)), k.sl, k.cl);
    const h2_t p1 = __builtin_elementwise_fma(h2bits(and_or(y, cm.lo, cm.bias)), k.sl, k.cl);
    const h2_t p2 = __builtin_elementwise_fma(h2bits(and_or(x, cm.hi, cm.bias)), k.sh, k.ch);
    const h2_t p3 = __builtin_elementwise_fma(h2bits(and_or(y, cm.hi, cm.bias)), k.sh, k.ch);
    const u32x4_t v = {bits(p0), bits(p1), bits(p2), bits(p3)};
    return __builtin_bit_cast(h8_t, v);
}

__device__ __forceinline__ uint32_t dword_of(const uint4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Four MFMAs t = 4*half .. 4*half+3 of every accumulator tile.  sa = the half's operand
// stage ([t][i][lane]), sb = the wave's weight slice.
__device__ __forceinline__ void half_block(const uint8_t* sa, const uint8_t* sb, int half, int n, int g, int lane,
                                           f4_t (&D1)[kMS][kNS]) {
    const f4_t zero = {0.f, 0.f, 0.f, 0.f};
    const CodeMask cm = code_mask();
    uint4 q[kNS];
    ChunkK ck[kNS];
#pragma unroll
    for (int j = 0; j < kNS; ++j) {
        q[j] = lds_u4(sb + ((1 + 4 * half + g) * kNS + j) * 256 + n * 16);
        ck[j] = chunk_consts(lds_u4(sb + j * 256 + n * 16), g, half);
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        h8_t B[kNS];
#pragma unroll
        for (int j = 0; j < kNS; ++j) B[j] = b_operand(dword_of(q[j], tt), ck[j], cm);
#pragma unroll
        for (int i = 0; i < kMS; ++i) {
            const h8_t A = __builtin_bit_cast(h8_t, lds_u4(sa + ((tt * kMS + i) * 64 + lane) * 16));
#pragma unroll
            for (int j = 0; j < kNS; ++j)
                D1[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[j], (half == 0 && tt == 0) ? zero : D1[i][j],
                                                                  0, 0, 0);
        }
    }
}

// Min term and the per-super-block epilogue: acc += d * D1 - dmin * D2.
__device__ __forceinline__ void block_epilogue(const uint8_t* ssum, const uint8_t* sb, int n, int g, int lane,
                                               const f4_t (&D1)[kMS][kNS], f4_t (&acc)[kMS][kNS]) {
    const f4_t zero = {0.f, 0.f, 0.f, 0.f};
    float d[kNS], dm[kNS];
    u32x4_t bm[kNS];
#pragma unroll
    for (int j = 0; j < kNS; ++j) {
        const uint4 h = lds_u4(sb + j * 256 + n * 16);
        d[j] = f16_to_f32(h.x);
        dm[j] = f16_to_f32(h.x >> 16);
        bm[j] = min_operand(h, g);
    }
#pragma unroll
    for (int i = 0; i < kMS; ++i) {
        const bf8_t As = __builtin_bit_cast(bf8_t, lds_u4(ssum + (i * 64 + lane) * 16));
#pragma unroll
        for (int j = 0; j < kNS; ++j) {
            const f4_t D2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(As, __builtin_bit_cast(bf8_t, bm[j]), zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[i][j][r] = __builtin_fmaf(d[j], D1[i][j][r], acc[i][j][r]);
                acc[i][j][r] = __builtin_fmaf(-dm[j], D2[r], acc[i][j][r]);
            }
        }
    }
}

constexpr int kA0 = kChunkA / 2;            // operands of t = 0..3
constexpr int kA1 = kChunkA / 2 + kChunkS;  // operands of t = 4..7, then the sums
constexpr int kWaitAll = 0x0F70;            // s_waitcnt vmcnt(0)
constexpr int kWaitB = 0x0F70 | 9;          // vmcnt(9): the 9 weight-slice copies issued last may pend

__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_prefill_gemm(
    const uint8_t* __restrict__ W, int64_t N, int nsb, const uint8_t* __restrict__ ws,
    const int32_t* __restrict__ rexp, int M, uint16_t* __restrict__ Y, float* __restrict__ Yf, int mtiles, int ntiles) {
    // Separate LDS objects per stage, so that reads of one stage are not ordered behind
    // direct-to-LDS copies still in flight into another.
    __shared__ __align__(16) uint8_t sA0[kA0];
    __shared__ __align__(16) uint8_t sA1[kA1];
    __shared__ __align__(16) uint8_t sB0[kWaves * kSliceB];
    __shared__ __align__(16) uint8_t sB1[kWaves * kSliceB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar) for the copies
    const int n = lane & 15, g = lane >> 4;

    // workgroup -> tile: the XCD of a workgroup is wg % 8; workgroups that share a weight
    // tile (all mtiles of one ntile) get consecutive ids on one XCD
    const int nwg = mtiles * ntiles;
    const int wg = blockIdx.x;
    const int pid = (nwg % 8 == 0) ? (wg % 8) * (nwg / 8) + wg / 8 : wg;
    const int mt = pid % mtiles, nt = pid / mtiles;

    const int64_t rb = (int64_t)nsb * 144;
    const int64_t row0 = (int64_t)nt * kBN + 64 * w;
    const int64_t nv64 = N - row0;
    const int nvalid = nv64 <= 0 ? 0 : (nv64 >= 64 ? 64 : (int)nv64);
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W + (nvalid ? row0 * rb : 0), (uint32_t)(nvalid * rb));
    uint8_t* const b0 = sB0 + w * kSliceB;
    uint8_t* const b1 = sB1 + w * kSliceB;

    f4_t acc[kMS][kNS], D1[kMS][kNS];
#pragma unroll
    for (int i = 0; i < kMS; ++i)
#pragma unroll
        for (int j = 0; j < kNS; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

    const int64_t cbase = (int64_t)mt * nsb;
    dma_blocks(wr, (uint32_t)rb, 0, b0, lane);
    dma_chunk<kA0 / 1024 / kWaves>(ws, cbase, 0, sA0, w, lane);
    // One super-block: [wait, h1 copy, next blocks] h0 MFMAs [wait, next h0 copy] h1 + epilogue.
#define AIPU_SUPERBLOCK(BCUR, BNXT)                                                                         \
    {                                                                                                       \
        __builtin_amdgcn_s_waitcnt(kWaitAll);                                                               \
        __syncthreads();                                                                                    \
        dma_chunk<kA1 / 1024 / kWaves>(ws, cbase + b, kA0, sA1, w, lane);                                   \
        const bool more = b + 1 < nsb;                                                                      \
        if (more) dma_blocks(wr, (uint32_t)rb, b + 1, BNXT, lane);                                          \
        half_block(sA0, BCUR, 0, n, g, lane, D1);                                                           \
        if (more) __builtin_amdgcn_s_waitcnt(kWaitB); else __builtin_amdgcn_s_waitcnt(kWaitAll);            \
        __syncthreads();                                                                                    \
        if (more) dma_chunk<kA0 / 1024 / kWaves>(ws, cbase + b + 1, 0, sA0, w, lane);                       \
        half_block(sA1, BCUR, 1, n, g, lane, D1);                                                           \
        block_epilogue(sA1 + kChunkA / 2, BCUR, n, g, lane, D1, acc);                                       \
    }
    for (int b = 0; b < nsb; ++b) {
        AIPU_SUPERBLOCK(b0, b1)
        if (++b >= nsb) break;
        AIPU_SUPERBLOCK(b1, b0)
    }
#undef AIPU_SUPERBLOCK

    // y = bf16(acc * 2^e_m); lane holds rows 16i + 4g + r, columns 16j + n
#pragma unroll
    for (int i = 0; i < kMS; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = (int64_t)mt * kBM + 16 * i + 4 * g + r;
            if (m >= M) continue;
            const int e = rexp[m];
#pragma unroll
            for (int j = 0; j < kNS; ++j) {
                const int col = 16 * j + n;
                if (col < nvalid) {
                    const float v = __builtin_ldexpf(acc[i][j][r], e);
                    Y[m * N + row0 + col] = (uint16_t)bf16_rne(v);
                    if (Yf) Yf[m * N + row0 + col] = v;
                }
            }
        }
    }
}

int64_t mpad(int64_t M) { return (M + kBM - 1) / kBM * kBM; }

}  // namespace

int64_t prefill_workspace_bytes(int64_t M, int64_t K) {
    return mpad(M) / kBM * (K / QK_K) * kChunk + mpad(M) * 4;
}

hipError_t launch_gemm_prefill(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                               uint16_t* y, float* y_f32, int precision, void* ws, hipStream_t st) {
    (void)precision;
    if (type != T_Q4_K || K % QK_K != 0 || K < QK_K || M < 1 || N < 1) return hipErrorInvalidValue;
    const int nsb = (int)(K / QK_K);
    const int64_t Mp = mpad(M);
    const int mtiles = (int)(Mp / kBM);
    const int64_t ntiles = (N + kBN - 1) / kBN;
    if ((int64_t)mtiles * ntiles > 0x7FFFFFFF || (int64_t)64 * nsb * 144 >= (1LL << 32)) return hipErrorInvalidValue;
    uint8_t* chunks = (uint8_t*)ws;
    int32_t* rexp = (int32_t*)(chunks + (int64_t)mtiles * nsb * kChunk);
    hipLaunchKernelGGL(k_prefill_rowexp, dim3((unsigned)(Mp / 4)), dim3(256), 0, st, x, K, (int)M, (int)Mp, rexp);
    hipLaunchKernelGGL(k_prefill_pack, dim3((unsigned)nsb, (unsigned)mtiles), dim3(256), 0, st, x, K, (int)M, rexp,
                       chunks, nsb);
    hipLaunchKernelGGL(k_prefill_gemm, dim3((unsigned)(mtiles * ntiles)), dim3(kWaves * 64), 0, st,
                       (const uint8_t*)w, N, nsb, chunks, rexp, (int)M, y, y_f32, mtiles, (int)ntiles);
    return hipGetLastError();
}

}  // namespace aipu
