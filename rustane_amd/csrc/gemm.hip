// Prefill GEMM launch policy: tile shape per problem size. The kernel itself
// is in gemm_kernel.hpp.
#include "gemm_kernel.hpp"

namespace hb {

template <int FT, int TT, int WF, int WT, class Epi>
static hipError_t launch_tile(const f16* W, const f16* X, int N, int T, int K, const Epi& epi,
                              hipStream_t st, int splits = 1) {
  const int tiles = ((N + FT - 1) / FT) * ((T + TT - 1) / TT);
  const int nk = K / 64, kq = (nk + splits - 1) / splits;
  hipLaunchKernelGGL((gemm_nt_kernel<FT, TT, WF, WT, Epi>), dim3(tiles, splits), dim3(WF * WT * 64),
                     0, st, W, X, N, T, K, kq, epi);
  return hipGetLastError();
}

// Split-K reduction: v = P[0] + P[1] + ... + P[S-1] (in that order, so the
// result does not depend on scheduling), handed to the epilogue four features
// at a time. HBM/MALL-bound; every split's loads are in flight together.
template <class Epi>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ P, int S,
                                                            int T, int N, size_t stride, Epi epi) {
  constexpr int MAXS = GEMM_MAX_SPLITS;
  const size_t n4 = (size_t)T * N / 4;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const size_t e = i * 4;
    f32x4 part[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s)
      if (s < S) part[s] = *(const f32x4*)(P + s * stride + e);
    f32x4 v = part[0];
#pragma unroll
    for (int s = 1; s < MAXS; ++s)
      if (s < S) v += part[s];
    epi((int)(e / N), (int)(e % N), v);
  }
}

// Tile choice (measured on MI355X over the 7B-shape projections): the largest
// tile that still gives most CUs a tile. 256x256 (8 waves of 64x128) when it
// yields >= 160 tiles, then 256x128 (8 waves of 64x64), then 128x128
// (4 waves), else 64x128 (4 waves of 32x64).
//
// Long-K problems with few 256x256 tiles (Wo and W2 at 512 tokens: 32 tiles)
// instead split K over up to GEMM_MAX_SPLITS ranges of >= 8 slices so that
// ~256 workgroups run the efficient 256x256 tile; the partials go through the
// caller's scratch and splitk_reduce applies the epilogue.
static long ntiles(int N, int T, int ft, int tt) { return (long)((N + ft - 1) / ft) * ((T + tt - 1) / tt); }

int gemm_splits(int N, int T, int K) {
  const long t256 = ntiles(N, T, 256, 256);
  const int nk = K / 64;
  if (t256 >= 96 || nk < 32) return 1;
  int S = (int)std::min<long>(GEMM_MAX_SPLITS, 256 / t256);
  S = std::min(S, nk / 8);
  return S >= 2 ? S : 1;
}

template <class Epi>
static hipError_t launch_gemm(const f16* W, const f16* X, int N, int T, int K, const Epi& epi,
                              const GemmScratch* scr, hipStream_t st) {
  if ((long)N * K >= (1L << 31) || (long)T * K >= (1L << 31)) return hipErrorInvalidValue;
  const int S = scr ? gemm_splits(N, T, K) : 1;
  if (S > 1) {
    const size_t stride = (size_t)T * N;
    if (!scr->p || (size_t)S * stride > scr->floats) return hipErrorInvalidValue;
    const hipError_t e = launch_tile<256, 256, 4, 2>(W, X, N, T, K, EpiSplit{scr->p, N, stride}, st, S);
    if (e != hipSuccess) return e;
    const size_t n4 = stride / 4;
    const int grid = (int)std::min<size_t>((n4 + 255) / 256, 4096);
    hipLaunchKernelGGL((splitk_reduce_kernel<Epi>), dim3(grid), dim3(256), 0, st, scr->p, S, T, N,
                       stride, epi);
    return hipGetLastError();
  }
  if (ntiles(N, T, 256, 256) >= 160) return launch_tile<256, 256, 4, 2>(W, X, N, T, K, epi, st);
  if (ntiles(N, T, 256, 128) >= 160) return launch_tile<256, 128, 4, 2>(W, X, N, T, K, epi, st);
  if (ntiles(N, T, 128, 128) >= 200) return launch_tile<128, 128, 2, 2>(W, X, N, T, K, epi, st);
  return launch_tile<64, 128, 2, 2>(W, X, N, T, K, epi, st);
}

hipError_t gemm_store(const f16* W, const f16* X, int N, int T, int K, float* C, hipStream_t st) {
  return launch_gemm(W, X, N, T, K, EpiStore{C, N}, nullptr, st);
}
hipError_t gemm_residual(const f16* W, const f16* X, int N, int T, int K, const EpiResidual& e,
                         const GemmScratch* scr, hipStream_t st) {
  return launch_gemm(W, X, N, T, K, e, scr, st);
}
hipError_t gemm_swiglu(const f16* W, const f16* X, int N, int T, int K, const EpiSwiGLU& e,
                       hipStream_t st) {
  return launch_gemm(W, X, N, T, K, e, nullptr, st);
}
hipError_t gemm_logits(const f16* W, const f16* X, int N, int T, int K, const EpiLogits& e,
                       hipStream_t st) {
  return launch_gemm(W, X, N, T, K, e, nullptr, st);
}
hipError_t gemm_qkv(const f16* W, const f16* X, int N, int T, int K, const EpiQKV& e,
                    hipStream_t st) {
  return launch_gemm(W, X, N, T, K, e, nullptr, st);
}

}  // namespace hb
