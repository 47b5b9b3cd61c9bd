// Prefill GEMM (large M).  Interim implementation: the streaming GEMV in 4-row activation
// chunks (tolerance mode), pending the matrix-core tile.
#include "common.hpp"
#include "launch.hpp"

namespace aipu {

hipError_t launch_gemm_prefill(int type, const void* w, int64_t N, int64_t K, const uint16_t* x, int64_t M,
                               uint16_t* y, int precision, hipStream_t st) {
    (void)precision;
    return launch_gemv_fast(type, w, N, K, x, M, y, nullptr, st);
}

}  // namespace aipu
