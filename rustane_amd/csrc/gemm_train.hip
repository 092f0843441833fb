// Training GEMMs: weight gradients (with per-tile sums of squares), the
// SwiGLU backward and the per-head products.
#include "gemm_launch.hpp"

namespace hb {

hipError_t gemm_wgrad(const f16* W, const f16* X, int N, int T, int K, float* g, int ld,
                      bool accumulate, hipStream_t st, float scale, float* sq_out, int* sq_tiles) {
  if (N % 4 || ld < N || (long)N * K >= (1L << 31) || (long)T * K >= (1L << 31))
    return hipErrorInvalidValue;
  if (sq_out) {
    // with per-tile sums of squares: 128x128 tiles at short K, else 256x256
    if (!sq_tiles) return hipErrorInvalidValue;
    if (K <= 1024) {
      *sq_tiles = (int)ntiles(N, T, 128, 128);
      if (accumulate)
        return launch_tile<128, 128, 2, 2>(W, X, N, T, K, EpiAccumSq{g, ld, scale, sq_out}, st);
      return launch_tile<128, 128, 2, 2>(W, X, N, T, K, EpiStoreSq{g, ld, scale, sq_out}, st);
    }
    *sq_tiles = (int)ntiles(N, T, 256, 256);
    if (accumulate)
      return launch_tile<256, 256, 2, 2>(W, X, N, T, K, EpiAccumSq{g, ld, scale, sq_out}, st);
    return launch_tile<256, 256, 2, 2>(W, X, N, T, K, EpiStoreSq{g, ld, scale, sq_out}, st);
  }
  // short K (few tokens): the fp32 output traffic dominates, two 128x128
  // tiles per CU overlap one's epilogue with the other's main loop; longer K
  // is MFMA-bound and takes the usual tile choice
  if (K <= 1024 && ntiles(N, T, 128, 128) >= 2 * GEMM_CUS) {
    if (accumulate) return launch_tile<128, 128, 2, 2>(W, X, N, T, K, EpiAccum{g, ld, scale}, st);
    return launch_tile<128, 128, 2, 2>(W, X, N, T, K, EpiStore{g, ld, scale}, st);
  }
  if (accumulate) return launch_gemm(W, X, N, T, K, EpiAccum{g, ld, scale}, nullptr, st);
  return launch_gemm(W, X, N, T, K, EpiStore{g, ld, scale}, nullptr, st);
}
hipError_t gemm_silu_bwd(const f16* W, const f16* X, int N, int T, int K, const EpiSiluBwd& e,
                         hipStream_t st) {
  if (N != e.hidden || N % 4) return hipErrorInvalidValue;
  return launch_gemm(W, X, N, T, K, e, nullptr, st);
}
hipError_t gemm_heads(const f16* W, const f16* X, int N, int T, int K, const EpiHeads& e,
                      hipStream_t st) {
  if (N != e.H * e.hd || e.hd % 4 || e.rows < e.S) return hipErrorInvalidValue;
  return launch_gemm(W, X, N, T, K, e, nullptr, st);
}

}  // namespace hb
