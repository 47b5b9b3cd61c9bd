// Persistent Q4_K GEMV for 2 .. 8 activation rows (tolerance mode), K = 2048 R (R <= 3) and
// at most three 8-row tiles per workgroup: one weight pass serves every row.
//
// Workgroup.  One workgroup per CU owns tiles wg, wg + G, wg + 2G.  Wave NCW copies them into
// LDS round slots with direct-to-LDS buffer loads: a round is 9 loads of 64 lanes x 16 B = 1152
// bytes of each of the tile's 8 rows (block pairs 4k .. 4k+3), laid out chunk-major (16-byte
// chunk c of row r at 16 (8c + r)), and is posted to an LDS counter once its loads have landed.
// The copy schedule is a runtime loop with fixed vmcnt waits, so the wave's code stays small.
// Compute wave w owns block pair w (np = 4R waves) for every tile and every activation row.
//
// Two kernels share this plan and differ in how a set (8 tile rows x one block pair) meets the
// activation rows:
// - k_gemvmp (row pairs, the default fast mode): every output is formed exactly as in the
//   single-row kernels (codes, seeds, MFMA chains, epilogue, block sums, pair sums and the
//   balanced tree of mfma_gemv.hpp), so row m of a batch is bit-identical to the one-row launch
//   on that row -- a speculative-verify batch reproduces greedy decoding.  A wave stages its
//   pair of every row in LDS and runs the pair's codes against the rows two at a time.
// - k_gemvmd (dense, AIPU_MODE_FAST_DENSE): one MFMA per sub-block serves all eight rows, with
//   the activation operands held in registers.  Its sums run in another order, so a row agrees
//   with its one-row launch within the tolerance only (its bits still depend neither on the
//   other rows nor on its position in the batch).
#include "common.hpp"
#include "launch.hpp"
#include "mfma_gemv.hpp"
#include "persist.hpp"

namespace aipu {

using namespace mg;
using namespace pst;

namespace {

constexpr int kTR8 = 8;          // rows per tile
constexpr int kMaxRows = 8;      // activation rows per launch
constexpr int kMaxTT = 3;        // tiles per workgroup
constexpr int kMaxNp = 12;       // block pairs per row (K <= 6144)
constexpr int kLoads = 9;        // direct-to-LDS loads per round
constexpr uint32_t kRoundRow = 128u * kLoads;   // bytes of a row per round (4 block pairs)
constexpr uint32_t kSlot = kTR8 * kRoundRow;    // bytes of a round
constexpr int kReaders = 4;      // sets that read a round

constexpr uint32_t kStg = kStgBytes;   // staged pair: operand entries + 16 sub-block sums
// Row-pair kernel: four round slots, four rounds in flight.  Deeper rings (up to 12 slots with
// 7 rounds in flight where the staged rows leave room) measured no faster: the sets, not the
// copies, bound these launches.
constexpr int kRpNS = 4, kRpQ = 4;

// A operands of a set for two activation rows (A: MFMAs t = 0..3 from entries t, B: entries
// 4 + t), the rows staged at st0 on lanes 16g + 4g + h and st1 on lanes 16g + 4g + 2 + h; every
// other lane keeps its zeros.  Then both rows' sub-block sums of this lane's block and group.
__device__ __forceinline__ void read_rows(u32x4_t (&A)[4], u32x4_t (&B)[4], float2& as0, float2& as1, uint32_t st0,
                                          uint32_t st1, int g, int n, int h) {
    const int j = n - 4 * g;   // 0 .. 3 on the operand lanes
    const uint32_t aa = ((j >> 1) & 1 ? st1 : st0) + 32u * (uint32_t)g + 16u * (uint32_t)(j & 1);
    const uint32_t so = kStgSums + 8u * (uint32_t)(g * 2 + h);
    uint64_t saved;
    asm volatile(
        "s_mov_b64 %[sv], exec\n\t"
        "s_and_b64 exec, exec, %[mask]\n\t"
        "ds_read_b128 %[a0], %[aa]\n\t"
        "ds_read_b128 %[a1], %[aa] offset:144\n\t"
        "ds_read_b128 %[a2], %[aa] offset:288\n\t"
        "ds_read_b128 %[a3], %[aa] offset:432\n\t"
        "ds_read_b128 %[b0], %[aa] offset:576\n\t"
        "ds_read_b128 %[b1], %[aa] offset:720\n\t"
        "ds_read_b128 %[b2], %[aa] offset:864\n\t"
        "ds_read_b128 %[b3], %[aa] offset:1008\n\t"
        "s_mov_b64 exec, %[sv]\n\t"
        "ds_read_b64 %[s0], %[p0]\n\t"
        "ds_read_b64 %[s1], %[p1]\n\t"
        "s_waitcnt lgkmcnt(0)"
        : [a0] "+v"(A[0]), [a1] "+v"(A[1]), [a2] "+v"(A[2]), [a3] "+v"(A[3]), [b0] "+v"(B[0]), [b1] "+v"(B[1]),
          [b2] "+v"(B[2]), [b3] "+v"(B[3]), [s0] "=&v"(as0), [s1] "=&v"(as1), [sv] "=&s"(saved)
        : [aa] "v"(aa), [mask] "s"(diag_mask(4)), [p0] "v"(st0 + so), [p1] "v"(st1 + so)
        : "memory", "scc");   // s_and_b64 writes SCC
}

// R rounds per tile (K = 2048 R), M2 row pairs (2 M2 - 1 <= M <= 2 M2).
template <int R, int M2>
__global__ __launch_bounds__(64 * (4 * 3 + 1)) void k_gemvmp(const uint8_t* __restrict__ W, int64_t N,
                                                           const uint16_t* __restrict__ X, int M,
                                                           uint16_t* __restrict__ Y, float* __restrict__ Yf,
                                                           int64_t ys, int ntiles) {
    constexpr int np = 4 * R, nsb = 8 * R;
    constexpr uint32_t rb = R * kRoundRow;
    constexpr int NCW = np;
    constexpr int NS = kRpNS, Q = kRpQ;
    extern __shared__ __align__(16) uint8_t s_dyn[];   // ring | staged rows | pair sums
    __shared__ uint32_t s_cnt[kMaxTT * R], s_read[kMaxTT * R], s_done[kMaxTT];
    uint8_t* const s_ring = s_dyn;
    uint8_t* const s_stage = s_dyn + NS * kSlot;                             // [pair][row] kStg each
    float* const s_red = (float*)(s_stage + (uint32_t)np * 2 * M2 * kStg);    // [t][row m][tile row][pair]
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x, G = gridDim.x;
    const int T = (ntiles - wg + G - 1) / G;   // <= kMaxTT
    const int U = T * R;                        // rounds of this workgroup
    const int n = lane & 15, g = lane >> 4, h = n >> 3, r = n & 7;
    const uint32_t loff = (uint32_t)(lane & 7) * rb + 16u * (uint32_t)(lane >> 3);
    // round u: 9 loads of 128 B of each tile row into slot u % NS
    auto issue = [&](int u) {
        const int t = u / R, k = u - t * R;
        const int64_t r0 = (int64_t)(wg + t * G) * kTR8;
        const int nvalid = (int)(N - r0 < kTR8 ? N - r0 : kTR8);
        const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W + r0 * (int64_t)rb, (uint32_t)nvalid * rb);
        uint8_t* dst = s_ring + (uint32_t)(u % NS) * kSlot;
        const uint32_t off = loff + kRoundRow * (uint32_t)k;
#pragma unroll
        for (int j = 0; j < kLoads; ++j) lds_dma16<kNT>(wr, dst + 1024u * j, off + 128u * j);
    };
    for (int i = tid; i < kMaxTT * R; i += blockDim.x) s_cnt[i] = s_read[i] = 0u;
    if (tid < kMaxTT) s_done[tid] = 0u;
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // counters initialised

    if (w == NCW) {
        copy_ring<NS, Q, 1, kLoads, kReaders>(0, U, s_cnt, s_read, issue);   // ---- copy wave
        return;
    }

    // ---- compute wave w: owns pair p = w and stages it for every row
    const int p = w;
    {
        const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, (uint32_t)(M * nsb) * 512u);
        uint4 xv[2 * M2];
#pragma unroll
        for (int m = 0; m < 2 * M2; ++m)
            xv[m] = buf_load16(xr, m < M ? (uint32_t)m * (uint32_t)nsb * 512u + (uint32_t)p * 1024u + 16u * (uint32_t)lane : kOOB);
#pragma unroll
        for (int m = 0; m < 2 * M2; ++m) stage_pair(xv[m], s_stage + (uint32_t)(p * 2 * M2 + m) * kStg, lane);
    }
    const HdrSel hs = hdr_sel(g);
    const CodeK ck = code_k();
    const bool hb = h != 0;
    // operand registers: the reads write the diagonal lanes only, every other lane stays zero
    u32x4_t A[4], B[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) A[i] = B[i] = u32x4_t{0u, 0u, 0u, 0u};
    const uint32_t stw = lds_addr(s_stage) + (uint32_t)(p * 2 * M2) * kStg;   // this pair's rows
    int seen = -1;
    for (int t = 0; t < T; ++t) {
        const int u = t * R + (p >> 2);
        const uint32_t oh = 288u * (uint32_t)(p & 3) + 144u * (uint32_t)h;   // header of block 2p + h, within the round
        const uint32_t tl = lds_addr(s_ring) + (uint32_t)(u % NS) * kSlot + 16u * (uint32_t)r;
        const uint32_t ah = tl + 8u * oh, aq = tl + 8u * (oh + 16u + 32u * (uint32_t)g);
        u32x4_t hv, q0, q1;
        uint32_t cv;
        asm volatile(
            "ds_read_b32 %3, %6\n\t"
            "ds_read_b128 %0, %4\n\t"
            "ds_read_b128 %1, %5\n\t"
            "ds_read_b128 %2, %5 offset:128\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(hv), "=&v"(q0), "=&v"(q1), "=&v"(cv)
            : "v"(ah), "v"(aq), "v"(lds_addr(&s_cnt[u]))
            : "memory");
        if (seen < u && (uint32_t)__builtin_amdgcn_readfirstlane(cv) < 1u) {
            spin_ge(&s_cnt[u], 1u);
            asm volatile(
                "ds_read_b128 %0, %3\n\t"
                "ds_read_b128 %1, %4\n\t"
                "ds_read_b128 %2, %4 offset:128\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(hv), "=&v"(q0), "=&v"(q1)
                : "v"(ah), "v"(aq)
                : "memory");
        }
        seen = seen < u ? u : seen;
        lds_post(&s_read[u]);   // the weights are in registers: one reader fewer
        const uint32_t qd[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        u32x4_t cl[4], ch[4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            cl[tt] = codes_lo(qd[2 * tt], qd[2 * tt + 1], ck);
            ch[tt] = codes_hi(qd[2 * tt], qd[2 * tt + 1], ck);
        }
        const Hdr H = hdr_decode(make_uint4(hv.x, hv.y, hv.z, hv.w), hs);
        float* rt = s_red + t * (kMaxRows * kTR8 * kMaxNp);
        // rows in quads: four block terms, one transposed block sum (lane 16i + n: row 4q + i)
#pragma unroll
        for (int q = 0; q < (M2 + 1) / 2; ++q) {
            float bq[4];
#pragma unroll
            for (int pp = 0; pp < 2 && 2 * q + pp < M2; ++pp) {
                const int mp = 2 * q + pp;
                // rows 2mp and 2mp + 1 (a missing second row repeats the first; it is never stored)
                const int m1 = 2 * mp + 1 < M ? 2 * mp + 1 : 2 * mp;
                const uint32_t st0 = stw + (uint32_t)(2 * mp) * kStg, st1 = stw + (uint32_t)m1 * kStg;
                float2 as0, as1;
                read_rows(A, B, as0, as1, st0, st1, g, n, h);
                f32x4_t dlo, dhi;
                dlo[0] = dlo[1] = -kCodeBiasF * as0.x;
                dlo[2] = dlo[3] = -kCodeBiasF * as1.x;
                dhi[0] = dhi[1] = -kCodeBiasF * as0.y;
                dhi[2] = dhi[3] = -kCodeBiasF * as1.y;
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    dlo = mfma(A[tt], cl[tt], dlo);
                    dhi = mfma(B[tt], ch[tt], dhi);
                }
                // D[4g + 2m' + h][n] is row 2mp + m' of column n's block
                bq[2 * pp] = block_term(H, hb ? dlo[1] : dlo[0], hb ? dhi[1] : dhi[0], as0.x, as0.y);
                bq[2 * pp + 1] = block_term(H, hb ? dlo[3] : dlo[2], hb ? dhi[3] : dhi[2], as1.x, as1.y);
            }
            const float bs = 2 * q + 1 < M2 ? block_sum4(bq[0], bq[1], bq[2], bq[3]) : block_sum2(bq[0], bq[1]);
            // pair sum on lanes 16i + r: block 2p, then block 2p + 1 from lane 16i + r + 8
            const float b1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(bs), 0x108, 0xF, 0xF, false));
            const int i = 2 * q + 1 < M2 ? g : (g & 1);
            if (h == 0 && (2 * q + 1 < M2 || g < 2)) rt[((4 * q + i) * kTR8 + r) * kMaxNp + p] = bs + b1;   // (nsb is even)
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // pair sums written before the count
        if constexpr (M2 >= 3) {
            // Five rows or more: wave 0 reduces the tile once every pair is in.  Its pair sits in
            // the tile's first round, so it has time to spare, and the waves of the last round go
            // straight on instead of reducing rows first.
            lds_post(&s_done[t]);
            if (w != 0) continue;
            spin_ge(&s_done[t], (uint32_t)np);
        } else {
            // fewer rows: the tile's last wave reduces it (cheaper than a waiting reducer)
            if (lds_add_rtn(&s_done[t]) != (uint32_t)np - 1u) continue;
        }
        // per row, v_k on lane 8 * tile row + k, then the tree
        const int rr = lane >> 3, k = lane & 7;
        const int64_t row = (int64_t)(wg + t * G) * kTR8 + rr;
        float v[2 * M2];
#pragma unroll
        for (int m = 0; m < 2 * M2; ++m) {
            const float* qp = rt + (m * kTR8 + rr) * kMaxNp;
            v[m] = k < np ? qp[k] : 0.0f;
#pragma unroll
            for (int j = 8; j < np; j += 8)
                if (k + j < np) v[m] += qp[k + j];
        }
#pragma unroll
        for (int m = 0; m < 2 * M2; ++m) {
            v[m] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[m]), 0xB1, 0xF, 0xF, false));
            v[m] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[m]), 0x4E, 0xF, 0xF, false));
            v[m] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[m]), 0x141, 0xF, 0xF, false));
        }
        if (k == 0 && row < N) {
#pragma unroll
            for (int m = 0; m < 2 * M2; ++m)
                if (m < M) {
                    Y[(int64_t)m * ys + row] = (uint16_t)bf16_rne(v[m]);
                    if (Yf) Yf[(int64_t)m * ys + row] = v[m];
                }
        }
    }
}

// Dense form: one MFMA per sub-block serves all eight activation rows.
//
// For sub-block j of block pair p (MFMA j = 0..7, lane l = 16 kq + n):
//   A row 2m + h (lane 16 kq + 2m + h) carries activation row m on block 2p + h: elements
//     8 kq .. 8 kq + 7 of sub-block j, in the element order of the codes (act_perm);
//   B column n = 8 h' + r carries the codes of the same elements of tile row r, block 2p + h':
//     qs bytes 32 (j / 2) + 8 kq .. + 7, low nibbles for even j, high nibbles for odd j;
// so D_j[2m + h'][n] = sum over sub-block j of a (128 + q) for activation row m, and lane
// 16 kq + n finds it for rows m = 2 kq (D register h') and 2 kq + 1 (register 2 + h').  The
// rows of A whose block differs from the column's are not used.
// Per lane and block:  y = d * sum_j sc_j D_j - sum_j (128 d sc_j + dmin m_j) S_j, with S_j the
// sub-block activation sum, which is sum_k a_k (d sc_j q_k - dmin m_j) (tools/q4k_ref.py:53-59).
// The activation operands (32 VGPRs) and the sums a lane needs (16) are loaded once and kept
// in registers for every tile, so the LDS holds only the weight ring and the pair sums.  The
// summation differs from the single-row kernels' (one 32-element product per sub-block instead
// of four 8-element ones, scales applied per sub-block), so a row agrees with its one-row
// launch within the tolerance, not bit for bit; a row's result does not depend on the other
// rows of the batch or on its position in it.
template <int R, int NS, int Q>
__global__ __launch_bounds__(64 * (4 * 3 + 1)) void k_gemvmd(const uint8_t* __restrict__ W, int64_t N,
                                                           const uint16_t* __restrict__ X, int M,
                                                           uint16_t* __restrict__ Y, float* __restrict__ Yf,
                                                           int64_t ys, int ntiles) {
    constexpr int np = 4 * R, nsb = 8 * R;
    constexpr uint32_t rb = R * kRoundRow;
    constexpr int NCW = np;
    extern __shared__ __align__(16) uint8_t s_dyn[];   // ring | pair sums
    __shared__ uint32_t s_cnt[kMaxTT * R], s_read[kMaxTT * R], s_done[kMaxTT];
    uint8_t* const s_ring = s_dyn;
    float* const s_red = (float*)(s_dyn + NS * kSlot);   // [t][row m][tile row][pair]
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = blockIdx.x, G = gridDim.x;
    const int T = (ntiles - wg + G - 1) / G;   // <= kMaxTT
    const int U = T * R;                        // rounds of this workgroup
    const uint32_t loff = (uint32_t)(lane & 7) * rb + 16u * (uint32_t)(lane >> 3);
    auto issue = [&](int u) {
        const int t = u / R, k = u - t * R;
        const int64_t r0 = (int64_t)(wg + t * G) * kTR8;
        const int nvalid = (int)(N - r0 < kTR8 ? N - r0 : kTR8);
        const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W + r0 * (int64_t)rb, (uint32_t)nvalid * rb);
        uint8_t* dst = s_ring + (uint32_t)(u % NS) * kSlot;
        const uint32_t off = loff + kRoundRow * (uint32_t)k;
#pragma unroll
        for (int j = 0; j < kLoads; ++j) lds_dma16<kNT>(wr, dst + 1024u * j, off + 128u * j);
    };
    for (int i = tid; i < kMaxTT * R; i += blockDim.x) s_cnt[i] = s_read[i] = 0u;
    if (tid < kMaxTT) s_done[tid] = 0u;
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // counters initialised

    if (w == NCW) {
        copy_ring<NS, Q, 1, kLoads, kReaders>(0, U, s_cnt, s_read, issue);   // ---- copy wave
        return;
    }

    // ---- compute wave w: block pair p = w for every row of every tile
    const int p = w;
    const int kq = lane >> 4, n = lane & 15, hq = n >> 3, r = n & 7;
    u32x4_t A[8];
    float as0[8], as1[8];   // S_j of rows 2 kq and 2 kq + 1 on block 2p + hq
    {
        const int ar = lane & 15, am = ar >> 1, ah = ar & 1;
        const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, (uint32_t)(M * nsb) * 512u);
        const uint32_t xo = (uint32_t)am * (uint32_t)nsb * 512u + 512u * (uint32_t)(2 * p + ah) + 16u * (uint32_t)kq;
        uint4 xv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[j] = buf_load16(xr, am < M ? xo + 64u * (uint32_t)j : kOOB);
        const uint32_t ones = 0x3F803F80u;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            A[j] = act_perm(xv[j]);
            float s = dot2(xv[j].x, ones, 0.f);
            s = dot2(xv[j].y, ones, s);
            s = dot2(xv[j].z, ones, s);
            s = dot2(xv[j].w, ones, s);
            s = block_sum(s);   // row ar's sub-block sum, on every lane with lane & 15 == ar
            as0[j] = __shfl(s, 4 * kq + hq, 64);
            as1[j] = __shfl(s, 4 * kq + 2 + hq, 64);
        }
    }
    const CodeK ck = code_k();
    const bool hb = hq != 0;
    const f32x4_t z4 = {0.f, 0.f, 0.f, 0.f};
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    int seen = -1;
    for (int t = 0; t < T; ++t) {
        const int u = t * R + (p >> 2);
        const uint32_t oh = 288u * (uint32_t)(p & 3) + 144u * (uint32_t)hq;   // block 2p + hq within the round
        const uint32_t ah = lds_addr(s_ring) + (uint32_t)(u % NS) * kSlot + 16u * (uint32_t)r + 8u * oh;
        // qs byte 32c + 8kq of the block: chunk oh / 16 + 1 + 2c + kq / 2, byte 8 (kq & 1)
        const uint32_t aq = ah + 128u + 128u * (uint32_t)(kq >> 1) + 8u * (uint32_t)(kq & 1);
        u32x4_t hv;
        u32x2_t q0, q1, q2, q3;
        uint32_t cv;
        asm volatile(
            "ds_read_b32 %5, %7\n\t"
            "ds_read_b128 %0, %6\n\t"
            "ds_read_b64 %1, %8\n\t"
            "ds_read_b64 %2, %8 offset:256\n\t"
            "ds_read_b64 %3, %8 offset:512\n\t"
            "ds_read_b64 %4, %8 offset:768\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(hv), "=&v"(q0), "=&v"(q1), "=&v"(q2), "=&v"(q3), "=&v"(cv)
            : "v"(ah), "v"(lds_addr(&s_cnt[u])), "v"(aq)
            : "memory");
        if (seen < u && (uint32_t)__builtin_amdgcn_readfirstlane(cv) < 1u) {
            spin_ge(&s_cnt[u], 1u);
            asm volatile(
                "ds_read_b128 %0, %5\n\t"
                "ds_read_b64 %1, %6\n\t"
                "ds_read_b64 %2, %6 offset:256\n\t"
                "ds_read_b64 %3, %6 offset:512\n\t"
                "ds_read_b64 %4, %6 offset:768\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(hv), "=&v"(q0), "=&v"(q1), "=&v"(q2), "=&v"(q3)
                : "v"(ah), "v"(aq)
                : "memory");
        }
        seen = seen < u ? u : seen;
        lds_post(&s_read[u]);   // the weights are in registers: one reader fewer
        // scales and mins of sub-blocks 0..3 (sA, mA) and 4..7 (sB, mB), one per byte, as in
        // get_scale_min_k4 (tools/q4k_ref.py:27-37)
        const float d = f16_to_f32(hv.x), dm = f16_to_f32(hv.x >> 16);
        const uint32_t sA = hv.y & 0x3F3F3F3Fu, mA = hv.z & 0x3F3F3F3Fu;
        const uint32_t sB = (hv.w & 0x0F0F0F0Fu) | ((hv.y >> 2) & 0x30303030u);
        const uint32_t mB = ((hv.w >> 4) & 0x0F0F0F0Fu) | ((hv.z >> 2) & 0x30303030u);
        const uint32_t qd[8] = {q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
        const float d128 = 128.0f * d;
        float T0 = 0.f, T1 = 0.f, C0 = 0.f, C1 = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const f32x4_t dl = mfma(A[2 * c], codes_lo(qd[2 * c], qd[2 * c + 1], ck), z4);
            const f32x4_t dh = mfma(A[2 * c + 1], codes_hi(qd[2 * c], qd[2 * c + 1], ck), z4);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int j = 2 * c + e;
                const f32x4_t& D = e ? dh : dl;
                const uint32_t sw = j < 4 ? sA : sB, mw = j < 4 ? mA : mB;
                const float sc = (float)((sw >> (8 * (j & 3))) & 0xFFu);
                const float mn = (float)((mw >> (8 * (j & 3))) & 0xFFu);
                T0 = __builtin_fmaf(sc, hb ? D[1] : D[0], T0);
                T1 = __builtin_fmaf(sc, hb ? D[3] : D[2], T1);
                const float cj = __builtin_fmaf(d128, sc, dm * mn);
                C0 = __builtin_fmaf(cj, as0[j], C0);
                C1 = __builtin_fmaf(cj, as1[j], C1);
            }
        }
        const float y0 = __builtin_fmaf(d, T0, -C0), y1 = __builtin_fmaf(d, T1, -C1);
        // pair sum on lanes 16 kq + r: block 2p, then block 2p + 1 from lane 16 kq + r + 8
        const float p0 = y0 + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y0), 0x108, 0xF, 0xF, false));
        const float p1 = y1 + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y1), 0x108, 0xF, 0xF, false));
        float* rt = s_red + t * (kMaxRows * kTR8 * kMaxNp);
        if (hq == 0) {
            rt[((2 * kq) * kTR8 + r) * kMaxNp + p] = p0;
            rt[((2 * kq + 1) * kTR8 + r) * kMaxNp + p] = p1;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // pair sums written before the count
        if (lds_add_rtn(&s_done[t]) != (uint32_t)np - 1u) continue;   // the tile's last wave reduces it
        // lane 8 m + tile row: the row's np pair sums (contiguous), added pairwise in a fixed tree
        const int m = lane >> 3, rr = lane & 7;
        const int64_t row = (int64_t)(wg + t * G) * kTR8 + rr;
        const float4* qp = (const float4*)(rt + (m * kTR8 + rr) * kMaxNp);
        float v;
        {
            const float4 a = qp[0];
            v = (a.x + a.y) + (a.z + a.w);
            if constexpr (np >= 8) {
                const float4 b = qp[1];
                v += (b.x + b.y) + (b.z + b.w);
            }
            if constexpr (np >= 12) {
                const float4 c = qp[2];
                v += (c.x + c.y) + (c.z + c.w);
            }
        }
        if (m < M && row < N) {
            Y[(int64_t)m * ys + row] = (uint16_t)bf16_rne(v);
            if (Yf) Yf[(int64_t)m * ys + row] = v;
        }
    }
}

int cus_m() {
    static int c = 0;
    if (c == 0) {
        int dev = 0, v = 0;
        c = hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                ? v : 256;
    }
    return c;
}

// dense kernel: every round keeps its own slot (at most three tiles of three rounds)
constexpr int kDnsNS = kMaxTT * 3, kDnsQ = 3;

size_t lds_bytes_dense() { return (size_t)kDnsNS * kSlot + (size_t)kMaxTT * kMaxRows * kTR8 * kMaxNp * 4; }

// row-pair kernel: the ring, the pairs staged for 2 M2 rows, the pair sums
size_t lds_bytes_pairs(int R, int M2) {
    return (size_t)kRpNS * kSlot + (size_t)(4 * R) * 2 * M2 * kStg + (size_t)kMaxTT * kMaxRows * kTR8 * kMaxNp * 4;
}

template <int R>
hipError_t run_md(const uint8_t* W, int64_t N, const uint16_t* x, int M, uint16_t* y, float* yf, int64_t ys, int G,
                  int ntiles, hipStream_t st) {
    hipLaunchKernelGGL((k_gemvmd<R, kDnsNS, kDnsQ>), dim3(G), dim3(64 * (4 * R + 1)), lds_bytes_dense(), st, W, N, x, M, y,
                       yf, ys, ntiles);
    return hipGetLastError();
}

template <int R, int M2>
hipError_t run_mp(const uint8_t* W, int64_t N, const uint16_t* x, int M, uint16_t* y, float* yf, int64_t ys, int G,
                  int ntiles, hipStream_t st) {
    hipLaunchKernelGGL((k_gemvmp<R, M2>), dim3(G), dim3(64 * (4 * R + 1)), lds_bytes_pairs(R, M2), st, W, N, x, M, y, yf,
                       ys, ntiles);
    return hipGetLastError();
}

}  // namespace

// The persistent multi-row GEMV serves K = 2048, 4096, 6144, 2..8 rows and N <= 3 * 8 * #CUs
// (at most three tiles per workgroup); the row-pair kernel also needs its staged rows to fit
// the LDS (they do at every such shape: 161,280 of 163,840 bytes at K = 6144, M = 8).
bool gemv_persist_m_supported(int64_t N, int64_t K, int64_t M, bool dense) {
    if (M < 2 || M > kMaxRows || N < 1 || K % 2048 != 0 || K < 2048 || K > 6144) return false;
    const int64_t ntiles = (N + kTR8 - 1) / kTR8;
    if (ntiles > (int64_t)kMaxTT * cus_m()) return false;
    return dense || lds_bytes_pairs((int)(K / 2048), (int)((M + 1) / 2)) <= 160u * 1024u;
}

hipError_t launch_gemv_persist_m(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                                 float* yf, int64_t ys, bool dense, hipStream_t st) {
    if (!gemv_persist_m_supported(N, K, M, dense)) return hipErrorInvalidValue;
    const int ntiles = (int)((N + kTR8 - 1) / kTR8);
    const int tt = (ntiles + cus_m() - 1) / cus_m();   // tiles per workgroup (<= 3)
    const int G = (ntiles + tt - 1) / tt;
    const int R = (int)(K / 2048), m = (int)M;
    if (dense) {
        if (R == 1) return run_md<1>(W, N, x, m, y, yf, ys, G, ntiles, st);
        if (R == 2) return run_md<2>(W, N, x, m, y, yf, ys, G, ntiles, st);
        return run_md<3>(W, N, x, m, y, yf, ys, G, ntiles, st);
    }
    const int M2 = (m + 1) / 2;
#define AIPU_MP(RV, MV) \
    if (R == RV && M2 == MV) return run_mp<RV, MV>(W, N, x, m, y, yf, ys, G, ntiles, st);
    AIPU_MP(1, 1) AIPU_MP(1, 2) AIPU_MP(1, 3) AIPU_MP(1, 4)
    AIPU_MP(2, 1) AIPU_MP(2, 2) AIPU_MP(2, 3) AIPU_MP(2, 4)
    AIPU_MP(3, 1) AIPU_MP(3, 2) AIPU_MP(3, 3) AIPU_MP(3, 4)
#undef AIPU_MP
    return hipErrorInvalidValue;
}

// Whether a bounded wait in this file's kernels gave up since the last call (then cleared).
hipError_t wait_gave_up_gemv_persist_m(uint32_t* flag) { return take_wait_gave_up(flag); }

}  // namespace aipu
