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
// Pre-pass (k_prefill_stage; k_prefill_rowexp + k_prefill_pack for K > 32768) writes the scaled activations into a caller
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
// Tiles.  Workgroup = 8 waves (two per SIMD) over a 128 x 256 (M x N) output tile; wave w
// owns all 128 activation rows (8 subtiles of 16) and weight rows 32w..32w+31 (2 subtiles):
// 16 accumulator tiles plus 16 per-super-block tiles, and each weight operand is built once
// per workgroup.  The two halves of a super-block's activation chunk and the weight blocks
// of the next super-block are copied into LDS while the current half computes; the barriers
// wait only for the copies a phase needs.  Workgroups sharing a weight tile are consecutive
// on one XCD (its L2 serves the re-reads).
#include "common.hpp"
#include "launch.hpp"

namespace aipu {

namespace {

constexpr int kBM = 128;                         // activation rows per workgroup
constexpr int kBN = 256;                         // weight rows per workgroup
constexpr int kWM = 1, kWN = 8;                  // waves along M and N
constexpr int kWaves = kWM * kWN;                // 8 waves: two per SIMD
constexpr int kMT = kBM / 16;                    // 16-row activation subtiles per workgroup tile
constexpr int kMS = kMT / kWM;                   // ... per wave
constexpr int kNS = kBN / kWN / 16;              // 16-row weight subtiles per wave
constexpr int kChunkA = 8 * kMT * 64 * 16;       // fp16 operands of one super-block
constexpr int kChunkS = kMT * 64 * 16;           // sum operands
constexpr int kChunk = kChunkA + kChunkS;        // 73728 B
static_assert(kChunkA / 2 % (1024 * kWaves) == 0 && (kChunkA / 2 + kChunkS) % (1024 * kWaves) == 0,
              "chunk halves must split into whole 1 KB copies per wave");

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

// The row exponent from the largest |x| bits of a row.
__device__ __forceinline__ int row_exponent(uint32_t mx) {
    int e = 0;
    if (mx != 0 && mx < 0x7F80u) {
        int ex;
        (void)frexpf(bf16_to_f32(mx), &ex);   // max = f * 2^ex, f in [0.5, 1)
        e = ex - 15;
    }
    return e;
}

// Row exponent e_m: the largest |x| of row m scaled by 2^-e_m lies in [2^14, 2^15).  Rows
// that are all zero, hold inf/nan, or lie past M get e = 0.  One workgroup per row.
__global__ __launch_bounds__(256) void k_prefill_rowexp(const uint16_t* __restrict__ X, int64_t K, int M,
                                                        int32_t* __restrict__ rexp) {
    __shared__ uint32_t part[4];
    const int row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    uint32_t mx = 0;
    if (row < M) {
        const uint16_t* xr = X + (int64_t)row * K;
#pragma unroll 4
        for (int64_t k = (int64_t)tid * 8; k < K; k += 2048) {
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
    if (lane == 0) part[tid >> 6] = mx;
    __syncthreads();
    if (tid == 0) rexp[row] = row_exponent(max(max(part[0], part[1]), max(part[2], part[3])));
}

// One (row, sub-block) item of chunk (mt, b): the 32 activations w (bf16 pairs, in K order)
// scaled by 2^-e into fp16, written into the 8-byte halves of the eight operand entries that
// carry them (sub-block s = 2c + hh sits in half hh of entries (t, g) with
// (t < 4 ? 0 : 2) + (g >> 1) = c), and their exactly split sum into half s >> 2 of the sum
// entry of lane group s & 3.  valid = false (rows past M) writes zeros.
__device__ __forceinline__ void pack_item(uint8_t* chunk, int i, int r, int s, const uint32_t (&w)[16], int e,
                                          bool valid) {
    uint32_t v[32];
    float sum = 0.f;
    if (valid) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            v[2 * k] = f16_scaled(w[k], e);
            v[2 * k + 1] = f16_scaled(w[k] >> 16, e);
        }
#pragma unroll
        for (int k = 0; k < 32; ++k) sum += __half2float(__ushort_as_half((unsigned short)v[k]));
    } else {
#pragma unroll
        for (int k = 0; k < 32; ++k) v[k] = 0;
    }
    const int c = s >> 1, hh = s & 1;
    const int t0 = c < 2 ? 0 : 4, gb = 2 * (c & 1);
#pragma unroll
    for (int g1 = 0; g1 < 2; ++g1) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const int base = 16 * g1 + 4 * tt;   // K offset inside the sub-block
            const uint2 o = make_uint2(v[base] | v[base + 2] << 16, v[base + 1] | v[base + 3] << 16);
            const int lane = 16 * (gb + g1) + r;
            *(uint2*)(chunk + ((int64_t)((t0 + tt) * kMT + i) * 64 + lane) * 16 + 8 * hh) = o;
        }
    }
    uint32_t h = 0, md = 0, l = 0;
    if (valid) split3(sum, h, md, l);
    *(uint2*)(chunk + kChunkA + ((int64_t)i * 64 + 16 * (s & 3) + r) * 16 + 8 * (s >> 2)) = make_uint2(h | md << 16, l);
}

__device__ __forceinline__ void load_item(const uint16_t* X, int64_t K, int m, int item, uint32_t (&w)[16]) {
    const uint4* src = (const uint4*)(X + (int64_t)m * K + 32 * (int64_t)item);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 x = src[q];
        w[4 * q] = x.x;
        w[4 * q + 1] = x.y;
        w[4 * q + 2] = x.z;
        w[4 * q + 3] = x.w;
    }
}

// Chunk (mt, b) of the workspace, one thread per (row, sub-block s), with the row exponents
// of k_prefill_rowexp (any K).
__global__ __launch_bounds__(256) void k_prefill_pack(const uint16_t* __restrict__ X, int64_t K, int M,
                                                      const int32_t* __restrict__ rexp, uint8_t* __restrict__ ws,
                                                      int nsb) {
    const int b = blockIdx.x, mt = blockIdx.y;
    const int item = blockIdx.z * 256 + threadIdx.x;   // 0 .. kBM * 8 - 1
    const int ml = item >> 3, s = item & 7;
    const int m = mt * kBM + ml;
    uint32_t w[16];
    const bool valid = m < M;
    if (valid) load_item(X, K, m, 8 * b + s, w);
    pack_item(ws + ((int64_t)mt * nsb + b) * kChunk, ml >> 4, ml & 15, s, w, valid ? rexp[m] : 0, valid);
}

// Both staging steps in one pass (K <= kStageMaxK): one workgroup per kStageRows padded rows,
// IPT items per thread.  Item j is (row j % kStageRows, sub-block j / kStageRows of the row),
// so the 64 items of a wave write kStageRows neighbouring rows of each operand entry.  Each
// thread loads its items' activations once, the workgroup takes each row's maximum of |x|
// bits (the same maximum, so the same exponent, as k_prefill_rowexp), and each thread packs
// its items as k_prefill_pack does.
constexpr int kStageRows = 4;
constexpr int kStageMaxIpt = 4;
constexpr int64_t kStageMaxK = 1024 * kStageMaxIpt / (8 * kStageRows) * QK_K;
template <int IPT>
__global__ __launch_bounds__(1024) void k_prefill_stage(const uint16_t* __restrict__ X, int64_t K, int M,
                                                        int32_t* __restrict__ rexp, uint8_t* __restrict__ ws,
                                                        int nsb) {
    constexpr int RW = kStageRows;
    __shared__ uint32_t part[16][RW];
    const int t = threadIdx.x, lane = t & 63, T = (int)blockDim.x;   // T: a multiple of 64
    const int m = blockIdx.x * RW + t % RW;                            // the row of every item of t
    const int nitems = RW * 8 * nsb;
    const bool valid = m < M;
    uint32_t w[IPT][16];
    uint32_t mx = 0;
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int j = t + k * T;
        if (j < nitems && valid) {
            load_item(X, K, m, j / RW, w[k]);
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                mx = max(mx, w[k][q] & 0x7FFFu);
                mx = max(mx, (w[k][q] >> 16) & 0x7FFFu);
            }
        }
    }
#pragma unroll
    for (int d = RW; d < 64; d <<= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, d, 64));
    if (lane < RW) part[t >> 6][lane] = mx;
    __syncthreads();
    mx = 0;
    for (int v = 0; v < T / 64; ++v) mx = max(mx, part[v][t % RW]);
    const int e = row_exponent(mx);
    if (t < RW) rexp[m] = e;
    const int mt = m / kBM, ml = m % kBM;
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int j = t + k * T;
        if (j < nitems) {
            const int g = j / RW;   // sub-block of the row
            pack_item(ws + ((int64_t)mt * nsb + g / 8) * kChunk, ml >> 4, ml & 15, g & 7, w[k], e, valid);
        }
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

// The weight rows of wave column wn (kNS subtiles of 16), super-block b, into their LDS
// slice, laid out [q][j][n] by 16-B piece q of the block (0 = header, 1 + p = qs piece p),
// row 16j + n: a lane group reading one piece of 16 rows touches 256 contiguous bytes.
// Ten pieces per row (piece 9, the first 16 B past the block, is never read) make a whole
// number of 1 KB copies per wave, so every wave's copy count and waits are static.
constexpr int kBpieces = 10;
constexpr int kSliceB = kBpieces * kNS * 256;  // bytes per wave column
constexpr int kBq = kSliceB / 1024;            // copies per wave per super-block
static_assert(kSliceB % 1024 == 0, "weight slice must be whole 1 KB copies");
__device__ __forceinline__ void dma_blocks(__amdgpu_buffer_rsrc_t wr, uint32_t rb, int b, uint8_t* slice, int lane) {
#pragma unroll
    for (int k = 0; k < kBq; ++k) {
        const int p = 64 * k + lane;                     // piece index in the slice
        const int q = p / (16 * kNS), row = p % (16 * kNS);
        dma16(wr, slice + k * 1024, (uint32_t)row * rb + (uint32_t)b * 144u + 16u * (uint32_t)q);
    }
}

// Workgroup barrier for LDS phases: waits for this wave's LDS reads and writes only.  The
// direct-to-LDS copies a phase needs are waited for explicitly (vmcnt) before it, so copies
// for later phases stay in flight across the barrier (__syncthreads would wait for all).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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
// so the masks sit in SGPRs and the bias in a VGPR the caller keeps live, all hidden from
// constant folding (which would split the and-or into two literal-operand instructions).
// The and-or itself is ordinary code, so the compiler's hazard checks around the matrix
// instructions see it.
struct CodeMask {
    uint32_t lo, hi;   // 0x000F000F, 0x00F000F0 (SGPR)
    uint32_t bias;     // 0x64006400 (VGPR): fp16 1024 in both halves
};

__device__ __forceinline__ CodeMask code_mask() {
    CodeMask c;
    c.lo = 0x000F000Fu;
    c.hi = 0x00F000F0u;
    c.bias = 0x64006400u;
    asm volatile("" : "+s"(c.lo));
    asm volatile("" : "+s"(c.hi));
    asm volatile("" : "+v"(c.bias));
    return c;
}

__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t bias) { return (v & mask) | bias; }

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
__device__ __forceinline__ void half_block(const uint8_t* sa, const uint8_t* sb, int half, int i0, int n, int g,
                                           int lane, f4_t (&D1)[kMS][kNS]) {
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
        // all kMS operand reads of the step go out before the B build and the MFMAs, so their
        // LDS latency overlaps that work instead of stalling every other MFMA pair
        h8_t A[kMS];
#pragma unroll
        for (int i = 0; i < kMS; ++i) A[i] = __builtin_bit_cast(h8_t, lds_u4(sa + ((tt * kMT + i0 + i) * 64 + lane) * 16));
        h8_t B[kNS];
#pragma unroll
        for (int j = 0; j < kNS; ++j) B[j] = b_operand(dword_of(q[j], tt), ck[j], cm);
#pragma unroll
        for (int i = 0; i < kMS; ++i) {
#pragma unroll
            for (int j = 0; j < kNS; ++j)
                D1[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[i], B[j], (half == 0 && tt == 0) ? zero : D1[i][j],
                                                                  0, 0, 0);
        }
    }
}

// Min term and the per-super-block epilogue: acc += d * D1 - dmin * D2.
__device__ __forceinline__ void block_epilogue(const uint8_t* ssum, const uint8_t* sb, int i0, int n, int g, int lane,
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
        const bf8_t As = __builtin_bit_cast(bf8_t, lds_u4(ssum + ((i0 + i) * 64 + lane) * 16));
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
constexpr int kWaitAll = 0x0F70;            // s_waitcnt vmcnt(0); | n gives vmcnt(n), n < 16

__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_prefill_gemm(
    const uint8_t* __restrict__ W, int64_t N, int nsb, const uint8_t* __restrict__ ws,
    const int32_t* __restrict__ rexp, int M, uint16_t* __restrict__ Y, float* __restrict__ Yf, int mtiles, int ntiles) {
    // Separate LDS objects per stage, so that reads of one stage are not ordered behind
    // direct-to-LDS copies still in flight into another.
    __shared__ __align__(16) uint8_t sA0[kA0];
    __shared__ __align__(16) uint8_t sA1[kA1];
    __shared__ __align__(16) uint8_t sB0[kWN * kSliceB];
    __shared__ __align__(16) uint8_t sB1[kWN * kSliceB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (scalar) for the copies
    const int wn = w;
    const int n = lane & 15, g = lane >> 4;
    const int i0 = 0;

    // workgroup -> tile: the XCD of a workgroup is wg % 8; workgroups that share a weight
    // tile (all mtiles of one ntile) get consecutive ids on one XCD
    const int nwg = mtiles * ntiles;
    const int wg = blockIdx.x;
    const int pid = (nwg % 8 == 0) ? (wg % 8) * (nwg / 8) + wg / 8 : wg;
    const int mt = pid % mtiles, nt = pid / mtiles;

    const int64_t rb = (int64_t)nsb * 144;
    constexpr int kRows = 16 * kNS;   // weight rows per wave
    const int64_t row0 = (int64_t)nt * kBN + kRows * wn;
    const int64_t nvr = N - row0;
    const int nvalid = nvr <= 0 ? 0 : (nvr >= kRows ? kRows : (int)nvr);
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W + (nvalid ? row0 * rb : 0), (uint32_t)(nvalid * rb));
    uint8_t* const b0 = sB0 + wn * kSliceB;
    uint8_t* const b1 = sB1 + wn * kSliceB;

    f4_t acc[kMS][kNS], D1[kMS][kNS];
#pragma unroll
    for (int i = 0; i < kMS; ++i)
#pragma unroll
        for (int j = 0; j < kNS; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

    const int64_t cbase = (int64_t)mt * nsb;
    dma_blocks(wr, (uint32_t)rb, 0, b0, lane);
    dma_chunk<kA0 / 1024 / kWaves>(ws, cbase, 0, sA0, w, lane);
    // One super-block: [wait, barrier, copy h1, copy next blocks] h0 MFMAs [wait for h1,
    // barrier, copy next h0] h1 MFMAs + epilogue.
#define AIPU_SUPERBLOCK(BCUR, BNXT)                                                                         \
    {                                                                                                       \
        __builtin_amdgcn_s_waitcnt(kWaitAll);                                                               \
        lds_barrier();                                                                                      \
        dma_chunk<kA1 / 1024 / kWaves>(ws, cbase + b, kA0, sA1, w, lane);                                   \
        dma_blocks(wr, (uint32_t)rb, bn, BNXT, lane);                                                   \
        half_block(sA0, BCUR, 0, i0, n, g, lane, D1);                                                       \
        __builtin_amdgcn_s_waitcnt(kWaitAll | kBq);                                                         \
        lds_barrier();                                                                                      \
        dma_chunk<kA0 / 1024 / kWaves>(ws, cbase + bn, 0, sA0, w, lane);                                    \
        half_block(sA1, BCUR, 1, i0, n, g, lane, D1);                                                       \
        block_epilogue(sA1 + kChunkA / 2, BCUR, i0, n, g, lane, D1, acc);                                   \
    }
    // The copies for super-block b + 1 are issued unconditionally (the last super-block
    // re-copies itself into the idle stages), so every wave's copy count and wait is static.
    for (int b = 0; b < nsb; ++b) {
        int bn = b + 1 < nsb ? b + 1 : b;
        AIPU_SUPERBLOCK(b0, b1)
        if (++b >= nsb) break;
        bn = b + 1 < nsb ? b + 1 : b;
        AIPU_SUPERBLOCK(b1, b0)
    }
#undef AIPU_SUPERBLOCK

    // y = bf16(acc * 2^e_m); lane holds rows 16(i0 + i) + 4g + r, columns 16j + n
#pragma unroll
    for (int i = 0; i < kMS; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t m = (int64_t)mt * kBM + 16 * (i0 + i) + 4 * g + r;
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
    if (K <= kStageMaxK) {
        const int items = kStageRows * 8 * nsb;
        const dim3 grid((unsigned)(Mp / kStageRows));
        const auto threads = [&](int ipt) { return dim3((unsigned)((items + 64 * ipt - 1) / (64 * ipt) * 64)); };
        if (items <= 1024)
            hipLaunchKernelGGL(k_prefill_stage<1>, grid, threads(1), 0, st, x, K, (int)M, rexp, chunks, nsb);
        else if (items <= 2048)
            hipLaunchKernelGGL(k_prefill_stage<2>, grid, threads(2), 0, st, x, K, (int)M, rexp, chunks, nsb);
        else
            hipLaunchKernelGGL(k_prefill_stage<kStageMaxIpt>, grid, threads(kStageMaxIpt), 0, st, x, K, (int)M, rexp,
                               chunks, nsb);
    } else {
        hipLaunchKernelGGL(k_prefill_rowexp, dim3((unsigned)Mp), dim3(256), 0, st, x, K, (int)M, rexp);
        hipLaunchKernelGGL(k_prefill_pack, dim3((unsigned)nsb, (unsigned)mtiles, kBM * 8 / 256), dim3(256), 0, st, x, K,
                           (int)M, rexp, chunks, nsb);
    }
    hipLaunchKernelGGL(k_prefill_gemm, dim3((unsigned)(mtiles * ntiles)), dim3(kWaves * 64), 0, st,
                       (const uint8_t*)w, N, nsb, chunks, rexp, (int)M, y, y_f32, mtiles, (int)ntiles);
    return hipGetLastError();
}

}  // namespace aipu
