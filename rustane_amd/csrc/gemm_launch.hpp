// Prefill GEMM launch policy: tile shape per problem size and split-K.
// Included by the translation units that instantiate the products (gemm.hip,
// gemm_qkv.hip, gemm_ffn.hip, gemm_train.hip: one per group of epilogues, so
// that they compile in parallel); the kernel is in gemm_kernel.hpp.
#pragma once
#include "gemm_kernel.hpp"

namespace hb {

// kw: W's row length; K (the X row length and the reduction length) is kw,
// or 2 * kw for split X rows (gemm_kernel.hpp). 0 means K.
template <int FT, int TT, int WF, int WT, class Epi>
static hipError_t launch_tile(const f16* W, const f16* X, int N, int T, int K, const Epi& epi,
                              hipStream_t st, int splits = 1, GemmBatch bt = {}, int kw = 0) {
  const int tiles = ((N + FT - 1) / FT) * ((T + TT - 1) / TT);
  const int nk = K / 64, kq = (nk + splits - 1) / splits;
  if (kw == 0) kw = K;
  if (nk < 1 || K % 64 || splits < 1 || (splits - 1) * kq >= nk) return hipErrorInvalidValue;
  if ((kw != K && 2 * kw != K) || kw % 64) return hipErrorInvalidValue;
  if (bt.n < 1 || bt.n > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemm_nt_kernel<FT, TT, WF, WT, Epi>), dim3(tiles, splits, bt.n),
                     dim3(WF * WT * 64), 0, st, W, X, N, T, K, kw, kq, epi, bt.wbs, bt.xbs);
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

// Tile choice: maximise (relative per-tile throughput) x (tiles per CU-round
// of the 256 CUs). All tiles run 4 waves (2x2); relative throughputs are
// measured on MI355X with whole rounds of tiles (7B shapes at 4096 tokens):
// 256x256 1.00, 192x256 0.93, 128x256 0.92, 192x128 0.88, 256x128 0.87,
// 128x128 0.77, 64x128 0.48. At 512 tokens this picks 192x256 for W1|W3
// (230 tiles), 192x128 for QKV (256 tiles) and 256x256 for the logits; at
// 4096 tokens 256x256 throughout.
//
// Long-K problems with few output tiles (Wo and W2 at 512 tokens: 128 tiles of
// 128x128) instead split K over up to GEMM_MAX_SPLITS ranges of >= 8 slices so
// that ~256 workgroups run; the partials go through the caller's scratch and
// splitk_reduce applies the epilogue. Measured GEMM time at 512 tokens, 7B
// shapes: Wo 25.5 us (128x128 x 2 splits) against 26.3 us (256x128 x 4) and
// 32.6 us unsplit; W2 57.7 us (128x128 x 2) against 53.2 us (256x128 x 4) and
// 79.5 us unsplit. Two splits halve the partial-sum traffic of the reduce;
// the long-K residual + norm projections (W2) still take 256x128 x 4
// (gemm_norm_splits), where the GEMM's gain outweighs the larger reduce.
// K from 1024 splits too (600M shape, Wo with K = 1536 at 512 tokens: 96
// workgroups of 64x128 unsplit, 144 of 128x128 in 3 splits; the batch-1
// forward 2.28 -> 2.16 ms).
constexpr int GEMM_CUS = 256;  // MI355X compute units
inline long ntiles(int N, int T, int ft, int tt) { return (long)((N + ft - 1) / ft) * ((T + tt - 1) / tt); }

// Widest feature tile an epilogue is instantiated for (Epi::kMaxFT, default
// 256): the attention-backward products have N = hd <= 128 features.
template <class E, class = void>
struct EpiMaxFT {
  static constexpr int value = 256;
};
template <class E>
struct EpiMaxFT<E, std::void_t<decltype(E::kMaxFT)>> {
  static constexpr int value = E::kMaxFT;
};

template <class Epi>
static hipError_t launch_gemm(const f16* W, const f16* X, int N, int T, int K, const Epi& epi,
                              const GemmScratch* scr, hipStream_t st, GemmBatch bt = {}, int kw = 0) {
  if ((long)N * K >= (1L << 31) || (long)T * K >= (1L << 31)) return hipErrorInvalidValue;
  if (bt.n != 1 && scr) return hipErrorInvalidValue;
  const int S = scr ? gemm_splits(N, T, K, scr->wgs) : 1;
  if (S > 1) {
    const size_t stride = (size_t)T * N;
    if (!scr->p || (size_t)S * stride > scr->floats) return hipErrorInvalidValue;
    const hipError_t e = launch_tile<128, 128, 2, 2>(W, X, N, T, K, EpiSplit{scr->p, N, stride}, st, S, {}, kw);
    if (e != hipSuccess) return e;
    const size_t n4 = stride / 4;
    const int grid = (int)std::min<size_t>((n4 + 255) / 256, 4096);
    hipLaunchKernelGGL((splitk_reduce_kernel<Epi>), dim3(grid), dim3(256), 0, st, scr->p, S, T, N,
                       stride, epi);
    return hipGetLastError();
  }
  // rel: throughput per CU of each tile shape with every CU busy (7B shapes at
  // 4096 tokens, time per full round of workgroups per tile area, 256x256 = 1);
  // the score weighs it by tiles per CU-round, where a partly filled last round
  // counts 0.4 + 0.6 x its fill (its tiles run faster with fewer neighbours:
  // fitted to the measured 7B launches at 512 and 4096 tokens).
  struct Cand {
    int ft, tt;
    float rel;
  };
  static constexpr Cand cands[] = {{256, 256, 1.00f}, {192, 256, 0.93f}, {128, 256, 0.92f},
                                   {192, 128, 0.88f}, {256, 128, 0.87f}, {128, 128, 0.77f},
                                   {64, 128, 0.48f}};
  int best = 0;
  float best_score = -1.f;
  constexpr int max_ft = EpiMaxFT<Epi>::value;
  for (int i = 0; i < (int)(sizeof(cands) / sizeof(cands[0])); ++i) {
    if (cands[i].ft > max_ft) continue;
    // batched (attention) products: no tile wider than the features rounded to 64
    if (bt.n > 1 && cands[i].ft > std::max(64, (N + 63) / 64 * 64)) continue;
    const long n = ntiles(N, T, cands[i].ft, cands[i].tt) * bt.n;
    const float fill = (float)(n % GEMM_CUS) / GEMM_CUS;
    const float rounds = (float)(n / GEMM_CUS) + (fill > 0.f ? 0.4f + 0.6f * fill : 0.f);
    const float score = cands[i].rel * (float)n / (rounds * GEMM_CUS);
    if (score > best_score + 1e-6f) {
      best_score = score;
      best = i;
    }
  }
  if constexpr (max_ft >= 256) {
    if (best == 0) return launch_tile<256, 256, 2, 2>(W, X, N, T, K, epi, st, 1, bt, kw);
    if (best == 4) return launch_tile<256, 128, 2, 2>(W, X, N, T, K, epi, st, 1, bt, kw);
  }
  if constexpr (max_ft >= 192) {
    if (best == 1) return launch_tile<192, 256, 2, 2>(W, X, N, T, K, epi, st, 1, bt, kw);
    if (best == 3) return launch_tile<192, 128, 2, 2>(W, X, N, T, K, epi, st, 1, bt, kw);
  }
  if (best == 2) return launch_tile<128, 256, 2, 2>(W, X, N, T, K, epi, st, 1, bt, kw);
  if (best == 5) return launch_tile<128, 128, 2, 2>(W, X, N, T, K, epi, st, 1, bt, kw);
  return launch_tile<64, 128, 2, 2>(W, X, N, T, K, epi, st, 1, bt, kw);
}

}  // namespace hb
