// Persistent single-row Q4_K GEMV (tolerance mode) for K <= 8192: the M = 1 hot path, also run
// with two activation rows (MR = 2, K <= 6144; below) and with the FFN half's RMSNorm in front
// (NORM).
//
// Workgroup.  One workgroup per CU owns TT tiles of 8 rows (tiles wg, wg + G, ...), G =
// #tiles / TT workgroups.  Wave NCW copies the tiles into LDS with direct-to-LDS buffer loads
// (16 B per lane, 1 KB of consecutive row bytes per instruction) in rounds of 1 KB per row,
// keeps Q rounds in flight and posts each round to an LDS counter as it lands.  The copy
// schedule is unrolled at compile time, so every vmcnt wait is static and no wait drains the
// whole pipeline.  Compute waves 0 .. NCW-1 own block pairs: wave w owns pairs w, w + NCW
// (XPW of them), stages those pairs' activations itself and keeps their block-diagonal MFMA
// operands in registers for the whole kernel; for every tile it computes its pairs (8 rows x
// 2 blocks, one MFMA set) as soon as the round holding them has landed.  Compute wave 0
// reduces each tile once all its pairs are in and stores the 8 outputs (the workgroup's last
// tile: the wave whose set completes it); the copy wave reuses a tile buffer once that tile is
// reduced (NB buffers).  The copy wave issues its first Q
// rounds before it joins the workgroup barrier.
//
// MFMA set (v_mfma_f32_16x16x32_bf16, lane 16g + n): column n = row n & 7 of the tile, block
// 2p + (n >> 3) of the pair; K-group g = qs bytes 32g .. 32g+31 of the block (sub-blocks 2g,
// 2g+1).  A rows 4g + h carry block 2p + h's activations on group g, so D[4g + h][n] is the
// sub-block sum of column n for h = n >> 3.  With MR = 2 rows, A rows 4g + 2m + hh carry row m of
// block 2p + hh (D register 2m + h holds row m's sum).  Codes, seeds and epilogue are those of
// mfma_gemv.hpp, and the reduction follows its fast-mode order: block terms (block_sum),
// pair sums (a row shift by 8), then the balanced tree over the pairs with three cross-lane
// adds -- bit-identical to the canon_sum of the small-batch kernels (k_gemvs, k_gemvm).
#include "common.hpp"
#include "launch.hpp"
#include "mfma_gemv.hpp"
#include "norm.hpp"
#include "persist.hpp"

namespace aipu {

using namespace mg;
using namespace pst;

namespace {

constexpr int kPR = 8;            // rows per tile
constexpr int kPMaxCW = 12;       // compute waves per workgroup
constexpr int kPMaxTT = 8;        // tiles per workgroup
constexpr int kPMaxNsb = 32;      // K <= 8192
constexpr int kPMaxPairs = kPMaxNsb / 2;
constexpr int kPStage = kStgBytes; // per pair: operand entries + 16 sub-block sums

// The FFN half's pre-FFN RMSNorm applied inside the router launch (NORM = true): compute wave
// w's pair p (elements 512p .. 512p + 511) is exactly wave p of the separate fast RMSNorm, so
// each wave forms that wave's sum of squares, the waves meet through LDS, and every wave
// takes the total in norm.hpp's order and scales its own pair before staging it.  Workgroup 0
// writes the normalised vector to `out` for the expert legs.  The bits equal the separate
// RMSNorm's, and the logits those of this kernel on its output.
struct NormIn {
    const uint16_t* gamma;
    uint32_t inv_len_bits;
    uint16_t* out;
};

// R rounds per tile (ceil(row bytes / 1 KB)), TT tiles per workgroup, XPW pairs per compute
// wave.  nsb = K / 256 is a runtime value with ceil(144 * nsb / 1024) == R.  COPY_ONLY = true
// is a measurement variant (aipu_measure_gemv): the copy wave runs the same copy schedule and
// the compute waves leave after the first barrier, so nothing is computed or written.
template <int R, int TT, int XPW, bool COPY_ONLY = false, bool NORM = false, int MR = 1>
__global__ __launch_bounds__(64 * (kPMaxCW + 1)) void k_gemv1p(const uint8_t* __restrict__ W, int64_t N, int nsb,
                                                             const uint16_t* __restrict__ X, uint16_t* __restrict__ Y,
                                                             float* __restrict__ Yf, int ntiles, NormIn nm, int64_t ys) {
    static_assert(MR == 1 || (MR == 2 && XPW == 1 && !NORM && !COPY_ONLY), "two rows: one pair per wave");
    constexpr int NB = TT < 3 ? TT : 3;                        // tile buffers
    // rounds in flight: up to 4; with buffer reuse (TT > NB) at most (NB - 1) R + 1 (see the
    // reuse wait), without it at most the TT R rounds there are
    constexpr int QL = TT <= NB ? TT * R : (NB - 1) * R + 1;
    constexpr int Q = 4 < QL ? 4 : QL;
    static_assert(Q >= 1 && 8 * Q <= 63, "rounds in flight within vmcnt");
    extern __shared__ __align__(16) uint8_t s_tile[];          // NB * 8 * pitch (direct-to-LDS targets only)
    __shared__ __align__(16) uint8_t s_stage[kPMaxPairs * kPStage * MR];     // [pair][row]
    __shared__ __align__(16) float s_red[NB * MR * kPR * kPMaxPairs];         // [buffer][row][tile row][pair]
    __shared__ uint32_t s_cnt[TT * R];                          // rounds landed
    __shared__ uint32_t s_done[TT];                             // pairs finished per tile
    __shared__ uint32_t s_freed[TT];                            // tile reduced, buffers free
    __shared__ float s_part[kNormWaves];                        // NORM: the waves' sums of squares
    __shared__ uint32_t s_normc;                                // NORM: sums posted
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int NCW = (int)(blockDim.x >> 6) - 1;
    const int wg = blockIdx.x, G = gridDim.x;
    const int T = (ntiles - wg + G - 1) / G;                    // tiles of this workgroup
    const int np = (nsb + 1) >> 1;
    const uint32_t rb = (uint32_t)nsb * 144u;
    const uint32_t P = tile_pitch(rb);
    const uint32_t TB = kPR * P;
    for (int i = tid; i < TT * R; i += blockDim.x) s_cnt[i] = 0u;
    if (tid < TT) {
        s_done[tid] = 0u;
        s_freed[tid] = 0u;
    }
    if (NORM && tid == 0) s_normc = 0u;

    // activation loads of the wave's own pairs go out before any weight copy
    uint4 xv[XPW], gv[XPW], xv1 = make_uint4(0u, 0u, 0u, 0u);
    if (w < NCW) {
        const __amdgpu_buffer_rsrc_t xr = buf_rsrc(X, (uint32_t)nsb * 512u);   // an odd nsb's last pair reads zeros
        if constexpr (MR == 2)   // the second row, X + K
            xv1 = buf_load16(buf_rsrc(X + (int64_t)nsb * 256, (uint32_t)nsb * 512u),
                             w < np ? (uint32_t)w * 1024u + 16u * (uint32_t)lane : kOOB);
        const __amdgpu_buffer_rsrc_t gr = buf_rsrc(nm.gamma, NORM ? (uint32_t)nsb * 512u : 0u);
#pragma unroll
        for (int i = 0; i < XPW; ++i) {
            const int p = w + NCW * i;
            xv[i] = buf_load16(xr, p < np ? (uint32_t)p * 1024u + 16u * (uint32_t)lane : kOOB);
            if constexpr (NORM) gv[i] = buf_load16(gr, p < np ? (uint32_t)p * 1024u + 16u * (uint32_t)lane : kOOB);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // the copy wave joins the barrier after issuing its first Q rounds (before its first post)
    if (w != NCW) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // counters initialised
    if constexpr (COPY_ONLY) {
        if (w != NCW) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // no load still in flight when the wave ends
            return;
        }
    }

    if (w == NCW) {
        // ---- copy wave: round u = t * R + k, posted in order once landed
        const uint32_t last = rb - 1024u * (R - 1);             // bytes per row in the last round
        uint32_t cnt0 = lds_addr(s_cnt);
        asm volatile("" : "+v"(cnt0));                           // a runtime base (see lds_post)
        constexpr int U = TT * R;
        static_for<0, U + Q - 1>([&](auto sI) {
            constexpr int step = decltype(sI)::value;
            if constexpr (step < U) {
                constexpr int t = step / R, k = step - t * R;
                // A buffer is reused once its previous tile is reduced.  That tile's last
                // round is posted by now: Q <= (NB - 1) * R + 1 keeps it at least Q rounds back.
                if constexpr (k == 0 && t >= NB && !COPY_ONLY) spin_ge(&s_freed[t - NB], 1u);
                const int64_t r0 = (int64_t)(wg + t * G) * kPR;
                const int nvalid = t < T ? (int)(N - r0 < kPR ? N - r0 : kPR) : 0;
                const __amdgpu_buffer_rsrc_t wr =
                    buf_rsrc(W + (nvalid > 0 ? r0 * (int64_t)rb : 0), (uint32_t)(nvalid > 0 ? nvalid : 0) * rb);
                uint8_t* tb = s_tile + (uint32_t)(t % NB) * TB;
#pragma unroll
                for (int rr = 0; rr < kPR; ++rr)
                    if (k < R - 1 || 16u * (uint32_t)lane < last)
                        lds_dma16<kNT>(wr, tb + (uint32_t)rr * P + 1024u * k, (uint32_t)rr * rb + 1024u * k + 16u * (uint32_t)lane);
            }
            constexpr int pu = step - (Q - 1);
            if constexpr (pu == 0) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // counters initialised
            if constexpr (pu >= 0) {
                constexpr int after = (U - 1 < step ? U - 1 : step) - pu;   // rounds issued after pu
                __builtin_amdgcn_s_waitcnt(wait_vm(kPR * after));
                lds_post(cnt0 + 4u * (uint32_t)pu);
            }
        });
        return;
    }

    // ---- compute waves: stage the own pairs, keep their operands in registers
    if constexpr (NORM) {
        // pair p is wave p of the RMSNorm's reduction; pairs past the data (and waves past the
        // pairs) count as zero, as the RMSNorm's idle waves do
#pragma unroll
        for (int i = 0; i < XPW; ++i) {
            const int p = w + NCW * i;
            const float s = norm_wave_sum(norm_sq8(xv[i]));
            if (p < np && lane == 0) s_part[p] = s;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the sums written before the post
        lds_post(&s_normc);
        spin_ge(&s_normc, (uint32_t)NCW);
        const float tot = norm_final_sum(lane < np ? s_part[lane] : 0.0f);
        const float inv = norm_inv(__shfl(tot, 0, 64), nm.inv_len_bits);
#pragma unroll
        for (int i = 0; i < XPW; ++i) {
            const int p = w + NCW * i;
            xv[i] = norm_apply8(xv[i], gv[i], inv);
            const uint32_t e = (uint32_t)p * 512u + 8u * (uint32_t)lane;   // first element of the lane's 8
            if (wg == 0 && p < np && e < (uint32_t)nsb * 256u) *(uint4*)(nm.out + e) = xv[i];
        }
    }
    const int n = lane & 15, g = lane >> 4, h = n >> 3, r = n & 7;
    u32x4_t A[XPW][8];
    float2 as[XPW], as1 = float2{0.f, 0.f};   // as1: the second row's sums (MR = 2)
#pragma unroll
    for (int i = 0; i < XPW; ++i) {
#pragma unroll
        for (int t = 0; t < 8; ++t) A[i][t] = u32x4_t{0u, 0u, 0u, 0u};
        as[i] = float2{0.f, 0.f};
        const int p = w + NCW * i;
        if (p >= np) continue;
        if constexpr (MR == 2) {
            // both rows staged; A rows 4g + 2m + hh carry row m of block 2p + hh, so the diagonal
            // lanes 16g + 4g + j (j < 4) read row j >> 1's entries of block j & 1
            uint8_t* st0 = s_stage + (uint32_t)(2 * p) * kPStage;
            uint8_t* st1 = st0 + kPStage;
            stage_pair(xv[i], st0, lane);
            stage_pair(xv1, st1, lane);
            const int j = (n - 4 * g) & 3;
            const uint32_t aa = lds_addr((j >> 1) & 1 ? st1 : st0) + 32u * (uint32_t)g + 16u * (uint32_t)(j & 1);
            const uint32_t so = kStgSums + 8u * (uint32_t)(g * 2 + h);
            uint64_t saved;
            asm volatile(
                "s_waitcnt lgkmcnt(0)\n\t"
                "s_mov_b64 %[sv], exec\n\t"
                "s_and_b64 exec, exec, %[mask]\n\t"
                "ds_read_b128 %[a0], %[aa]\n\t"
                "ds_read_b128 %[a1], %[aa] offset:144\n\t"
                "ds_read_b128 %[a2], %[aa] offset:288\n\t"
                "ds_read_b128 %[a3], %[aa] offset:432\n\t"
                "ds_read_b128 %[a4], %[aa] offset:576\n\t"
                "ds_read_b128 %[a5], %[aa] offset:720\n\t"
                "ds_read_b128 %[a6], %[aa] offset:864\n\t"
                "ds_read_b128 %[a7], %[aa] offset:1008\n\t"
                "s_mov_b64 exec, %[sv]\n\t"
                "ds_read_b64 %[s0], %[p0]\n\t"
                "ds_read_b64 %[s1], %[p1]\n\t"
                "s_waitcnt lgkmcnt(0)"
                : [a0] "+v"(A[i][0]), [a1] "+v"(A[i][1]), [a2] "+v"(A[i][2]), [a3] "+v"(A[i][3]), [a4] "+v"(A[i][4]),
                  [a5] "+v"(A[i][5]), [a6] "+v"(A[i][6]), [a7] "+v"(A[i][7]), [s0] "=&v"(as[i]), [s1] "=&v"(as1),
                  [sv] "=&s"(saved)
                : [aa] "v"(aa), [mask] "s"(diag_mask(4)), [p0] "v"(lds_addr(st0) + so), [p1] "v"(lds_addr(st1) + so)
                : "memory", "scc");   // s_and_b64 writes SCC
            continue;
        }
        uint8_t* st = s_stage + (uint32_t)p * kPStage;
        stage_pair(xv[i], st, lane);
        // the operands (diagonal lanes 16g + 4g + h, h < 2) and this lane's sums
        const uint32_t aa = lds_addr(st) + 32u * (uint32_t)g + 16u * (uint32_t)((n - 4 * g) & 1);
        uint64_t saved;
        asm volatile(
            "s_waitcnt lgkmcnt(0)\n\t"
            "s_mov_b64 %[sv], exec\n\t"
            "s_and_b64 exec, exec, %[mask]\n\t"
            "ds_read_b128 %[a0], %[aa]\n\t"
            "ds_read_b128 %[a1], %[aa] offset:144\n\t"
            "ds_read_b128 %[a2], %[aa] offset:288\n\t"
            "ds_read_b128 %[a3], %[aa] offset:432\n\t"
            "ds_read_b128 %[a4], %[aa] offset:576\n\t"
            "ds_read_b128 %[a5], %[aa] offset:720\n\t"
            "ds_read_b128 %[a6], %[aa] offset:864\n\t"
            "ds_read_b128 %[a7], %[aa] offset:1008\n\t"
            "s_mov_b64 exec, %[sv]\n\t"
            "ds_read_b64 %[as], %[sa]\n\t"
            "s_waitcnt lgkmcnt(0)"
            : [a0] "+v"(A[i][0]), [a1] "+v"(A[i][1]), [a2] "+v"(A[i][2]), [a3] "+v"(A[i][3]), [a4] "+v"(A[i][4]),
              [a5] "+v"(A[i][5]), [a6] "+v"(A[i][6]), [a7] "+v"(A[i][7]), [as] "=&v"(as[i]), [sv] "=&s"(saved)
            : [aa] "v"(aa), [mask] "s"(diag_mask(2)), [sa] "v"(lds_addr(st) + kStgSums + 8u * (uint32_t)(g * 2 + h))
            : "memory", "scc");   // s_and_b64 writes SCC
    }
    const HdrSel hs = hdr_sel(g);
    const CodeK ck = code_k();
    int seen = -1;   // highest round known to have landed
    bool last_done = false;
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int i = 0; i < XPW; ++i) {
            const int p = w + NCW * i;
            if (p >= np) break;
            const uint32_t pend = 288u * (uint32_t)p + 287u < rb ? 288u * (uint32_t)p + 287u : rb - 1u;
            const int u = t * R + (int)(pend / 1024u);         // the round holding the pair's last byte
            const uint32_t blk = 2u * (uint32_t)p + (uint32_t)h;
            const uint32_t wrow = lds_addr(s_tile) + (uint32_t)(t % NB) * TB + (uint32_t)r * P + 144u * blk;
            // the round counter and the operands in one LDS batch: a posted counter proves that
            // the operands read after it (in DS order) had landed; otherwise wait and read again
            u32x4_t hv, q0, q1;
            uint32_t cv;
            asm volatile(
                "ds_read_b32 %3, %6\n\t"
                "ds_read_b128 %0, %4\n\t"
                "ds_read_b128 %1, %5\n\t"
                "ds_read_b128 %2, %5 offset:16\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(hv), "=&v"(q0), "=&v"(q1), "=&v"(cv)
                : "v"(wrow), "v"(wrow + 16u + 32u * (uint32_t)g), "v"(lds_addr(&s_cnt[u]))
                : "memory");
            if (seen < u && (uint32_t)__builtin_amdgcn_readfirstlane(cv) < 1u) {
                spin_ge(&s_cnt[u], 1u);
                asm volatile(
                    "ds_read_b128 %0, %3\n\t"
                    "ds_read_b128 %1, %4\n\t"
                    "ds_read_b128 %2, %4 offset:16\n\t"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(hv), "=&v"(q0), "=&v"(q1)
                    : "v"(wrow), "v"(wrow + 16u + 32u * (uint32_t)g)
                    : "memory");
            }
            seen = seen < u ? u : seen;
            f32x4_t dlo, dhi;
            dlo[0] = dlo[1] = -kCodeBiasF * as[i].x;
            dhi[0] = dhi[1] = -kCodeBiasF * as[i].y;
            if constexpr (MR == 2) {   // D[4g + 2m + hh][n]: row m's seeds in registers 2m, 2m + 1
                dlo[2] = dlo[3] = -kCodeBiasF * as1.x;
                dhi[2] = dhi[3] = -kCodeBiasF * as1.y;
            } else {
                dlo[2] = dlo[3] = dhi[2] = dhi[3] = 0.f;
            }
            const uint32_t qd[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                dlo = mfma(A[i][tt], codes_lo(qd[2 * tt], qd[2 * tt + 1], ck), dlo);
                dhi = mfma(A[i][4 + tt], codes_hi(qd[2 * tt], qd[2 * tt + 1], ck), dhi);
            }
            const Hdr H = hdr_decode(make_uint4(hv.x, hv.y, hv.z, hv.w), hs);
            float bt;
            if constexpr (MR == 2) {   // lane 16i + n: row i & 1's block sum (the additions of block_sum)
                const float t0 = block_term(H, h ? dlo[1] : dlo[0], h ? dhi[1] : dhi[0], as[i].x, as[i].y);
                const float t1 = block_term(H, h ? dlo[3] : dlo[2], h ? dhi[3] : dhi[2], as1.x, as1.y);
                bt = block_sum2(t0, t1);
            } else {
                bt = block_sum(block_term(H, h ? dlo[1] : dlo[0], h ? dhi[1] : dhi[0], as[i].x, as[i].y));
            }
            // pair sum on lanes 16i + r (row r): block 2p, then block 2p+1 from lane 16i + r + 8
            const float b1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(bt), 0x108, 0xF, 0xF, false));
            const float ps = bt + (2 * p + 1 < nsb ? b1 : 0.0f);
            float* rt = s_red + (t % NB) * (MR * kPR * kPMaxPairs);
            if constexpr (MR == 2) {
                if (lane < 32 && (lane & 15) < kPR) rt[((lane >> 4) * kPR + (lane & 7)) * kPMaxPairs + p] = ps;
            } else {
                if (lane < kPR) rt[lane * kPMaxPairs + p] = ps;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // pair sums written before the count
            if (t == T - 1) last_done = lds_add_rtn(&s_done[t]) == (uint32_t)np - 1u;
            else lds_post(&s_done[t]);
        }
        // Wave 0 reduces a tile once every pair is in.  Its own pairs sit in the tile's first
        // round, so it has time to spare; the waves of the last round, whose sets finish a tile,
        // go straight on to the next tile.  The workgroup's last tile has no next tile: the wave
        // whose post completes it reduces it, with no wait.
        if (t == T - 1 ? last_done : w == 0) {
            if (t < T - 1) spin_ge(&s_done[t], (uint32_t)np);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float* rt = s_red + (t % NB) * (MR * kPR * kPMaxPairs) + m * (kPR * kPMaxPairs);
                // v_k on lane 8 * row + k, then the tree (xor 1, xor 2, mirror)
                const int rr = lane >> 3, k = lane & 7;
                float v = k < np ? rt[rr * kPMaxPairs + k] : 0.0f;
                for (int j = k + 8; j < np; j += 8) v += rt[rr * kPMaxPairs + j];
                v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
                v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
                v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
                const int64_t row = (int64_t)(wg + t * G) * kPR + rr;
                if (k == 0 && row < N) {
                    Y[m * ys + row] = (uint16_t)bf16_rne(v);
                    if (Yf) Yf[m * ys + row] = v;
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // reads of rt done before the buffer is reused
            lds_post(&s_freed[t]);
        }
    }
}

// Measurement: an empty kernel with k_gemv1p's launch shape (grid, block and LDS).
__global__ __launch_bounds__(64 * (kPMaxCW + 1)) void k_gemv1p_empty() {}

int cu_count() {
    static int n = 0;
    if (n == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            n = v;
        else
            n = 256;
    }
    return n;
}

template <int R, int XPW, bool COPY_ONLY = false, bool NORM = false>
hipError_t run_p(const uint8_t* W, int64_t N, int nsb, const uint16_t* x, uint16_t* y, float* yf, int TT, int G,
                 int ntiles, int ncw, size_t lds, hipStream_t st, NormIn nm = NormIn{nullptr, 0u, nullptr}) {
    const dim3 grid(G), block(64 * (ncw + 1));
    if constexpr (NORM) {   // the FFN half's router: at most two tiles per workgroup
        if (TT == 1)
            hipLaunchKernelGGL((k_gemv1p<R, 1, XPW, false, true>), grid, block, lds, st, W, N, nsb, x, y, yf, ntiles, nm,
                               (int64_t)0);
        else if (TT == 2)
            hipLaunchKernelGGL((k_gemv1p<R, 2, XPW, false, true>), grid, block, lds, st, W, N, nsb, x, y, yf, ntiles, nm,
                               (int64_t)0);
        else
            return hipErrorInvalidValue;
        return hipGetLastError();
    }
    switch (TT) {
#define AIPU_P(TV) \
    case TV: hipLaunchKernelGGL((k_gemv1p<R, TV, XPW, COPY_ONLY>), grid, block, lds, st, W, N, nsb, x, y, yf, ntiles, nm, \
                                (int64_t)0); break;
        AIPU_P(1)
        AIPU_P(2)
        AIPU_P(3)
        AIPU_P(4)
        AIPU_P(5)
        AIPU_P(6)
        AIPU_P(7)
        AIPU_P(8)
#undef AIPU_P
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Two activation rows (K <= 6144: one block pair per compute wave), at most four tiles per workgroup.
template <int R>
hipError_t run_p2(const uint8_t* W, int64_t N, int nsb, const uint16_t* x, uint16_t* y, float* yf, int64_t ys, int TT,
                  int G, int ntiles, int ncw, size_t lds, hipStream_t st) {
    const dim3 grid(G), block(64 * (ncw + 1));
    const NormIn nm{nullptr, 0u, nullptr};
    switch (TT) {
#define AIPU_P2(TV) \
    case TV: hipLaunchKernelGGL((k_gemv1p<R, TV, 1, false, false, 2>), grid, block, lds, st, W, N, nsb, x, y, yf, \
                                ntiles, nm, ys); break;
        AIPU_P2(1)
        AIPU_P2(2)
        AIPU_P2(3)
        AIPU_P2(4)
#undef AIPU_P2
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Launch plan of a one-row GEMV of N rows over K (K <= 8192).
struct PPlan {
    int nsb, ntiles, TT, G, R, np, xpw, ncw, nb;
    size_t lds;
};
PPlan p_plan(int64_t N, int64_t K) {
    PPlan q;
    q.nsb = (int)(K / QK_K);
    q.ntiles = (int)((N + kPR - 1) / kPR);
    const int cus = cu_count();
    q.TT = (q.ntiles + cus - 1) / cus;
    q.TT = q.TT > kPMaxTT ? kPMaxTT : q.TT;
    q.G = (q.ntiles + q.TT - 1) / q.TT;
    q.R = (144 * q.nsb + 1023) / 1024;
    q.np = (q.nsb + 1) / 2;
    q.xpw = q.np > kPMaxCW ? 2 : 1;
    q.ncw = (q.np + q.xpw - 1) / q.xpw;
    q.nb = q.TT < 3 ? q.TT : 3;
    q.lds = (size_t)q.nb * kPR * tile_pitch((uint32_t)q.nsb * 144u);
    return q;
}

}  // namespace

bool gemv_persist_supported(int64_t N, int64_t K) {
    return N >= 1 && K >= QK_K && K % QK_K == 0 && K / QK_K <= kPMaxNsb && N <= ((int64_t)1 << 31);
}

// y[0 .. N) = x . W^T for one activation row (Q4_K, K <= 8192).  variant 1: the copy schedule
// alone; variant 2: an empty kernel of the same launch shape (measurement only).
hipError_t launch_gemv_persist(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, uint16_t* y, float* yf,
                               hipStream_t st, int variant) {
    if (!gemv_persist_supported(N, K)) return hipErrorInvalidValue;
    const PPlan q = p_plan(N, K);
    const int nsb = q.nsb, ntiles = q.ntiles, TT = q.TT, G = q.G, R = q.R, xpw = q.xpw, ncw = q.ncw, nb = q.nb;
    const size_t lds = q.lds;
    if (variant == 2) {
        // the same dynamic LDS plus the kernel's static arrays
        const size_t stat = (size_t)kPMaxPairs * kPStage + (size_t)nb * kPR * kPMaxPairs * 4 + (size_t)TT * (R + 2) * 4;
        hipLaunchKernelGGL(k_gemv1p_empty, dim3(G), dim3(64 * (ncw + 1)), lds + stat, st);
        return hipGetLastError();
    }
    if (variant == 1) {
        switch (R * 4 + xpw) {
            case 1 * 4 + 1: return run_p<1, 1, true>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
            case 2 * 4 + 1: return run_p<2, 1, true>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
            case 3 * 4 + 1: return run_p<3, 1, true>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
            case 4 * 4 + 1: return run_p<4, 1, true>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
            case 4 * 4 + 2: return run_p<4, 2, true>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
            case 5 * 4 + 2: return run_p<5, 2, true>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
            default: return hipErrorInvalidValue;
        }
    }
    switch (R * 4 + xpw) {
        case 1 * 4 + 1: return run_p<1, 1>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
        case 2 * 4 + 1: return run_p<2, 1>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
        case 3 * 4 + 1: return run_p<3, 1>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
        case 4 * 4 + 1: return run_p<4, 1>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
        case 4 * 4 + 2: return run_p<4, 2>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
        case 5 * 4 + 2: return run_p<5, 2>(W, N, nsb, x, y, yf, TT, G, ntiles, ncw, lds, st);
        default: return hipErrorInvalidValue;
    }
}

bool gemv_persist_norm_supported(int64_t N, int64_t K) {
    return gemv_persist_supported(N, K) && p_plan(N, K).TT <= 2;
}

hipError_t launch_gemv_persist_norm(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, const uint16_t* gamma,
                                    uint32_t inv_len_bits, uint16_t* x_norm, uint16_t* y, hipStream_t st) {
    if (!gemv_persist_norm_supported(N, K)) return hipErrorInvalidValue;
    const PPlan q = p_plan(N, K);
    const NormIn nm{gamma, inv_len_bits, x_norm};
    const int nsb = q.nsb, ntiles = q.ntiles, TT = q.TT, G = q.G, ncw = q.ncw;
    switch (q.R * 4 + q.xpw) {
        case 1 * 4 + 1: return run_p<1, 1, false, true>(W, N, nsb, x, y, nullptr, TT, G, ntiles, ncw, q.lds, st, nm);
        case 2 * 4 + 1: return run_p<2, 1, false, true>(W, N, nsb, x, y, nullptr, TT, G, ntiles, ncw, q.lds, st, nm);
        case 3 * 4 + 1: return run_p<3, 1, false, true>(W, N, nsb, x, y, nullptr, TT, G, ntiles, ncw, q.lds, st, nm);
        case 4 * 4 + 1: return run_p<4, 1, false, true>(W, N, nsb, x, y, nullptr, TT, G, ntiles, ncw, q.lds, st, nm);
        case 4 * 4 + 2: return run_p<4, 2, false, true>(W, N, nsb, x, y, nullptr, TT, G, ntiles, ncw, q.lds, st, nm);
        case 5 * 4 + 2: return run_p<5, 2, false, true>(W, N, nsb, x, y, nullptr, TT, G, ntiles, ncw, q.lds, st, nm);
        default: return hipErrorInvalidValue;
    }
}

bool gemv_persist2_supported(int64_t N, int64_t K) {
    if (!gemv_persist_supported(N, K) || K > 6144) return false;
    return p_plan(N, K).TT <= 4;
}

// Rows 0 and 1 of x (row stride K) in one launch; row m of y at y + m * ys.  Each row is formed
// exactly as the one-row launch forms it (the same sets, block sums, pair sums and tree).
hipError_t launch_gemv_persist2(const uint8_t* W, int64_t N, int64_t K, const uint16_t* x, uint16_t* y, float* yf,
                                int64_t ys, hipStream_t st) {
    if (!gemv_persist2_supported(N, K)) return hipErrorInvalidValue;
    const PPlan q = p_plan(N, K);
    switch (q.R) {
        case 1: return run_p2<1>(W, N, q.nsb, x, y, yf, ys, q.TT, q.G, q.ntiles, q.ncw, q.lds, st);
        case 2: return run_p2<2>(W, N, q.nsb, x, y, yf, ys, q.TT, q.G, q.ntiles, q.ncw, q.lds, st);
        case 3: return run_p2<3>(W, N, q.nsb, x, y, yf, ys, q.TT, q.G, q.ntiles, q.ncw, q.lds, st);
        case 4: return run_p2<4>(W, N, q.nsb, x, y, yf, ys, q.TT, q.G, q.ntiles, q.ncw, q.lds, st);
        default: return hipErrorInvalidValue;
    }
}

// Whether a bounded wait in this file's kernels gave up since the last call (then cleared).
hipError_t wait_gave_up_gemv_persist(uint32_t* flag) { return take_wait_gave_up(flag); }

}  // namespace aipu
