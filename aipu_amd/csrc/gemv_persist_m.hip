// Persistent Q4_K GEMV for 2 .. 8 activation rows (tolerance mode), K = 2048 R (R <= 3) and
// at most three 8-row tiles per workgroup: one weight pass serves every row.
//
// Workgroup.  One workgroup per CU owns tiles wg, wg + G, wg + 2G.  Wave NCW copies them into
// a ring of LDS round slots with direct-to-LDS buffer loads: a round is 9 loads of 64 lanes x
// 16 B = 1152 bytes of each of the tile's 8 rows (block pairs 4k .. 4k+3), laid out chunk-
// major (16-byte chunk c of row r at 16 (8c + r)), up to four rounds in flight in four slots,
// each posted to an LDS counter once its loads have landed.  A slot is refilled once the 4 sets that read its round hold their weights in
// registers.  The copy schedule is a runtime loop with fixed vmcnt waits, so the wave's code
// stays small.
//
// Compute wave w owns block pair w (np = 4R waves).  It stages pair w of every activation row
// in LDS, and for every tile builds the pair's codes once (8 rows x 2 blocks) and runs them
// against the rows two at a time: A rows 4g + 2m' + h carry row 2mp + m' of block 2w + h on
// K-group g, so D[4g + 2m' + h][n] is the sub-block sum of column n for that row.  Every
// output is formed exactly as in the single-row kernels (codes, seeds, MFMA order, epilogue,
// block_sum, pair sum, the balanced tree over the pairs), so row m of a batch is bit-identical
// to the single-row launch on that row.  From five rows on, compute wave 0 reduces each tile
// once all its pairs are in; below that the tile's last wave does.
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
constexpr uint32_t kStg = kStgBytes;   // staged pair: operand entries + 16 sub-block sums
constexpr int kReaders = 4;      // sets that read a round
// Round slots and rounds in flight.  Deeper rings (up to 12 slots with 7 rounds in flight
// where the staged rows leave room) measured no faster here: the sets, not the copies, bound
// these launches.
__host__ __device__ constexpr int ring_slots(int) { return 4; }
__host__ __device__ constexpr int ring_depth(int) { return 4; }

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
    constexpr int NS = ring_slots(M2), Q = ring_depth(M2);
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
        if (seen < u && __builtin_amdgcn_readfirstlane(cv) < 1u) {
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

int cus_m() {
    static int c = 0;
    if (c == 0) {
        int dev = 0, v = 0;
        c = hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
                ? v : 256;
    }
    return c;
}

size_t lds_bytes(int R, int M2) {
    return (size_t)ring_slots(M2) * kSlot + (size_t)(4 * R) * 2 * M2 * kStg + (size_t)kMaxTT * kMaxRows * kTR8 * kMaxNp * 4;
}

template <int R, int M2>
hipError_t run_m(const uint8_t* W, int64_t N, const uint16_t* x, int M, uint16_t* y, float* yf, int64_t ys, int G,
                 int ntiles, hipStream_t st) {
    hipLaunchKernelGGL((k_gemvmp<R, M2>), dim3(G), dim3(64 * (4 * R + 1)), lds_bytes(R, M2), st, W, N, x, M, y, yf, ys, ntiles);
    return hipGetLastError();
}

}  // namespace

// The persistent multi-row GEMV serves K = 2048, 4096, 6144, 2..8 rows and N <= 3 * 8 * #CUs
// (at most three tiles per workgroup).
bool gemv_persist_m_supported(int64_t N, int64_t K, int64_t M) {
    if (M < 2 || M > kMaxRows || N < 1 || K % 2048 != 0 || K < 2048 || K > 6144) return false;
    const int64_t ntiles = (N + kTR8 - 1) / kTR8;
    return ntiles <= (int64_t)kMaxTT * cus_m() && lds_bytes((int)(K / 2048), (int)((M + 1) / 2)) <= 160u * 1024u;
}

hipError_t launch_gemv_persist_m(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, int64_t M, uint16_t* y,
                                 float* yf, int64_t ys, hipStream_t st) {
    if (!gemv_persist_m_supported(N, K, M)) return hipErrorInvalidValue;
    const int ntiles = (int)((N + kTR8 - 1) / kTR8);
    const int tt = (ntiles + cus_m() - 1) / cus_m();   // tiles per workgroup (<= 3)
    const int G = (ntiles + tt - 1) / tt;
    const int R = (int)(K / 2048), M2 = (int)((M + 1) / 2), m = (int)M;
#define AIPU_M(RV, MV) \
    if (R == RV && M2 == MV) return run_m<RV, MV>(W, N, x, m, y, yf, ys, G, ntiles, st);
    AIPU_M(1, 1) AIPU_M(1, 2) AIPU_M(1, 3) AIPU_M(1, 4)
    AIPU_M(2, 1) AIPU_M(2, 2) AIPU_M(2, 3) AIPU_M(2, 4)
    AIPU_M(3, 1) AIPU_M(3, 2) AIPU_M(3, 3) AIPU_M(3, 4)
#undef AIPU_M
    return hipErrorInvalidValue;
}

}  // namespace aipu
