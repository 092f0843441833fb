// Prefill GEMM launch policy: tile shape per problem size. The kernel itself
// is in gemm_kernel.hpp.
#include "gemm_kernel.hpp"

namespace hb {

template <int FT, int TT, int WF, int WT, class Epi>
static hipError_t launch_tile(const f16* W, const f16* X, int N, int T, int K, const Epi& epi,
                              hipStream_t st) {
  const int tiles = ((N + FT - 1) / FT) * ((T + TT - 1) / TT);
  hipLaunchKernelGGL((gemm_nt_kernel<FT, TT, WF, WT, Epi>), dim3(tiles), dim3(WF * WT * 64), 0,
                     st, W, X, N, T, K, epi);
  return hipGetLastError();
}

// Tile choice (measured on MI355X over the 7B-shape projections): the largest
// tile that still gives most CUs a tile. 256x256 (8 waves of 64x128) when it
// yields >= 160 tiles, then 256x128 (8 waves of 64x64), then 128x128
// (4 waves), else 64x128 (4 waves of 32x64) for small-N projections such as Wo
// and W2 at 512 tokens.
static long ntiles(int N, int T, int ft, int tt) { return (long)((N + ft - 1) / ft) * ((T + tt - 1) / tt); }

template <class Epi>
static hipError_t launch_gemm(const f16* W, const f16* X, int N, int T, int K, const Epi& epi,
                              hipStream_t st) {
  if ((long)N * K >= (1L << 31) || (long)T * K >= (1L << 31)) return hipErrorInvalidValue;
  if (ntiles(N, T, 256, 256) >= 160) return launch_tile<256, 256, 4, 2>(W, X, N, T, K, epi, st);
  if (ntiles(N, T, 256, 128) >= 160) return launch_tile<256, 128, 4, 2>(W, X, N, T, K, epi, st);
  if (ntiles(N, T, 128, 128) >= 200) return launch_tile<128, 128, 2, 2>(W, X, N, T, K, epi, st);
  return launch_tile<64, 128, 2, 2>(W, X, N, T, K, epi, st);
}

hipError_t gemm_store(const f16* W, const f16* X, int N, int T, int K, float* C, hipStream_t st) {
  return launch_gemm(W, X, N, T, K, EpiStore{C, N}, st);
}
hipError_t gemm_residual(const f16* W, const f16* X, int N, int T, int K, const EpiResidual& e,
                         hipStream_t st) {
  return launch_gemm(W, X, N, T, K, e, st);
}
hipError_t gemm_swiglu(const f16* W, const f16* X, int N, int T, int K, const EpiSwiGLU& e,
                       hipStream_t st) {
  return launch_gemm(W, X, N, T, K, e, st);
}
hipError_t gemm_logits(const f16* W, const f16* X, int N, int T, int K, const EpiLogits& e,
                       hipStream_t st) {
  return launch_gemm(W, X, N, T, K, e, st);
}
hipError_t gemm_qkv(const f16* W, const f16* X, int N, int T, int K, const EpiQKV& e,
                    hipStream_t st) {
  return launch_gemm(W, X, N, T, K, e, st);
}

}  // namespace hb
