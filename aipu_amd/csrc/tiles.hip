// Mixed-type tile GEMV: each tile is one ggml type over a contiguous range of output rows
// (the per-column w_type mux of src/glm_matmul_q4k.v:76-101 and the tile sequence of
// tools/q4k_mixed_gen.py:382-440).  Each tile is dispatched to its type's GEMV kernel on
// the same stream, writing its rows of y in place.
#include "common.hpp"
#include "launch.hpp"

namespace aipu {

hipError_t launch_gemv_tiles(const aipu_tile_desc* tiles, int n_tiles, int64_t N, int64_t K, const uint16_t* x,
                             int64_t M, uint16_t* y, float* y_f32, int mode, hipStream_t st) {
    // Row r of tile t lands in column row0 + r of every activation row m: the tile writes
    // an [M][nrows] block of the [M][N] output with row stride N, which the per-row
    // kernels express by running once per activation row.
    if (mode == AIPU_MODE_FAST) {
        // every tile in one launch, the activation rows in passes of up to four (gemv_mixed.hip)
        bool all = true;
        for (int t = 0; t < n_tiles; ++t) all = all && gemv_mixed_supported(tiles[t].ggml_type, K);
        if (all) return launch_gemv_mixed(tiles, n_tiles, K, x, M, y, y_f32, N, st);
    }
    for (int t = 0; t < n_tiles; ++t) {
        const aipu_tile_desc& d = tiles[t];
        if (mode == AIPU_MODE_FAST && d.ggml_type == T_Q4_K && gemv_mfma_supported(d.nrows, K, M)) {
            // the matrix-core GEMV writes all M rows of the tile's column slice directly
            const hipError_t e = launch_gemv_mfma(d.w, d.nrows, K, x, M, y + d.row0,
                                                  y_f32 ? y_f32 + d.row0 : nullptr, N, st);
            if (e != hipSuccess) return e;
            continue;
        }
        for (int64_t m = 0; m < M; ++m) {
            hipError_t e;
            uint16_t* ym = y + m * N + d.row0;
            float* yfm = y_f32 ? y_f32 + m * N + d.row0 : nullptr;
            if (mode == AIPU_MODE_FAST && (d.ggml_type == T_Q4_K || d.ggml_type == T_BF16))
                e = launch_gemv_fast(d.ggml_type, d.w, d.nrows, K, x + m * K, 1, ym, yfm, st);
            else
                e = launch_gemv_ref(d.ggml_type, d.w, d.nrows, K, x + m * K, 1, ym, yfm, st);
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

}  // namespace aipu
