// Prefill GEMM launch policy: tile shape per problem size. The kernel itself
// is in gemm_kernel.hpp.
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

// Split-K reduction fused with the RMSNorm that follows a residual projection
// (cpu/rmsnorm.rs:149-183): one workgroup of 256 threads per token row adds the
// splits in order, applies the residual epilogue (out = res + alpha * v), and
// normalises the row into xn. The element-to-thread mapping and the block sum
// are those of rmsnorm_kernel, so xn is bit-identical to reduce + rmsnorm.
template <int NPT>  // as rmsnorm_kernel: N = NPT * 1024 held in registers, or 0 = any N
__global__ __launch_bounds__(256) void splitk_reduce_norm_kernel(const float* __restrict__ P, int S,
                                                                 int N, size_t stride,
                                                                 EpiResidual e, NormOut no) {
  constexpr int MAXS = GEMM_MAX_SPLITS;
  __shared__ float red[4];
  const int t = blockIdx.x;
  const size_t row = (size_t)t * N;
  f16* orow = no.xn + (no.split ? 2 * row : row);
  const size_t lo = no.split ? (size_t)N : 0;  // split xn rows: [hi | lo]
  float ss = 0.f;
  if constexpr (NPT > 0) {
    f32x4 y[NPT], g[NPT];
    {
      f32x4 part[NPT][MAXS], r[NPT];
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const size_t c = row + threadIdx.x * 4 + i * 1024;
#pragma unroll
        for (int s = 0; s < MAXS; ++s)
          if (s < S) part[i][s] = *(const f32x4*)(P + s * stride + c);
        r[i] = *(const f32x4*)(e.res + c);
      }
#pragma unroll
      for (int i = 0; i < NPT; ++i) g[i] = *(const f32x4*)(no.gamma + threadIdx.x * 4 + i * 1024);
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        f32x4 v = part[i][0];
#pragma unroll
        for (int s = 1; s < MAXS; ++s)
          if (s < S) v += part[i][s];
        y[i].x = v.x * e.alpha + r[i].x;
        y[i].y = v.y * e.alpha + r[i].y;
        y[i].z = v.z * e.alpha + r[i].z;
        y[i].w = v.w * e.alpha + r[i].w;
        *(f32x4*)(e.out + row + threadIdx.x * 4 + i * 1024) = y[i];
        ss += y[i].x * y[i].x + y[i].y * y[i].y + y[i].z * y[i].z + y[i].w * y[i].w;
      }
    }
    ss = block_sum<4>(ss, red);
    const float rinv = 1.0f / sqrtf(ss * (1.0f / (float)N) + no.eps);
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      f32x4 o;
      o.x = y[i].x * rinv * g[i].x;
      o.y = y[i].y * rinv * g[i].y;
      o.z = y[i].z * rinv * g[i].z;
      o.w = y[i].w * rinv * g[i].w;
      store_f16x4(orow + threadIdx.x * 4 + i * 1024, o, lo);
    }
  } else {
    for (int c = threadIdx.x * 4; c < N; c += 1024) {
      f32x4 part[MAXS];
#pragma unroll
      for (int s = 0; s < MAXS; ++s)
        if (s < S) part[s] = *(const f32x4*)(P + s * stride + row + c);
      f32x4 v = part[0];
#pragma unroll
      for (int s = 1; s < MAXS; ++s)
        if (s < S) v += part[s];
      const f32x4 r = *(const f32x4*)(e.res + row + c);
      f32x4 y;
      y.x = v.x * e.alpha + r.x;
      y.y = v.y * e.alpha + r.y;
      y.z = v.z * e.alpha + r.z;
      y.w = v.w * e.alpha + r.w;
      *(f32x4*)(e.out + row + c) = y;
      ss += y.x * y.x + y.y * y.y + y.z * y.z + y.w * y.w;
    }
    ss = block_sum<4>(ss, red);
    const float rinv = 1.0f / sqrtf(ss * (1.0f / (float)N) + no.eps);
    for (int c = threadIdx.x * 4; c < N; c += 1024) {
      const f32x4 y = *(const f32x4*)(e.out + row + c);  // this thread's own stores
      const f32x4 g = *(const f32x4*)(no.gamma + c);
      f32x4 o;
      o.x = y.x * rinv * g.x;
      o.y = y.y * rinv * g.y;
      o.z = y.z * rinv * g.z;
      o.w = y.w * rinv * g.w;
      store_f16x4(orow + c, o, lo);
    }
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
static long ntiles(int N, int T, int ft, int tt) { return (long)((N + ft - 1) / ft) * ((T + tt - 1) / tt); }

int gemm_splits(int N, int T, int K, int wgs) {
  const long t = ntiles(N, T, 128, 128);
  const int nk = K / 64;
  if (t >= wgs || nk < 16) return 1;
  int S = (int)std::min<long>(GEMM_MAX_SPLITS, wgs / t);
  S = std::min(S, nk / 8);
  return S >= 2 ? S : 1;
}

// The residual + RMSNorm projections (gemm_residual_norm): a long reduction
// (K >= 2N) whose 256x128 tiles in S splits fill the wgs workgroups exactly
// runs on those tiles (7B W2 at 512 tokens: 64 tiles x 4 splits instead of
// 128 of 128x128 x 2; batch-1 forward 9.40-9.44 -> 9.34-9.36 ms: the wider
// tile reads each activation panel half as often per flop, which outweighs
// the reduce reading 4 partials instead of 2; Wo, K = N, gains less).
// Otherwise gemm_splits on 128x128 tiles. *wide tells which.
int gemm_norm_splits(int N, int T, int K, int wgs, bool* wide) {
  *wide = false;
  const int S = gemm_splits(N, T, K, wgs);
  if (S <= 1 || K < 2 * N) return S;
  const long t = ntiles(N, T, 256, 128);
  if (t <= 0 || wgs % t) return S;
  const int Sw = (int)(wgs / t);
  if (Sw < 2 || Sw > GEMM_MAX_SPLITS || Sw * 8 > K / 64) return S;
  *wide = true;
  return Sw;
}

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

hipError_t gemm_store(const f16* W, const f16* X, int N, int T, int K, float* C, hipStream_t st) {
  return launch_gemm(W, X, N, T, K, EpiStore{C, N}, nullptr, st);
}
hipError_t gemm_residual(const f16* W, const f16* X, int N, int T, int K, const EpiResidual& e,
                         const GemmScratch* scr, hipStream_t st, int kw) {
  return launch_gemm(W, X, N, T, K, e, scr, st, {}, kw);
}
hipError_t gemm_residual_norm(const f16* W, const f16* X, int N, int T, int K, const EpiResidual& e,
                              const NormOut& no, const GemmScratch* scr, hipStream_t st, int kw,
                              hipEvent_t mid) {
  if (e.ld != N) return hipErrorInvalidValue;
  bool wide = false;
  const int S = scr ? gemm_norm_splits(N, T, K, scr->wgs, &wide) : 1;
  hipError_t err2 = hipSuccess;
  if (S > 1) {
    const size_t stride = (size_t)T * N;
    if (!scr->p || (size_t)S * stride > scr->floats || (long)N * K >= (1L << 31)) return hipErrorInvalidValue;
    const hipError_t err =
        wide ? launch_tile<256, 128, 2, 2>(W, X, N, T, K, EpiSplit{scr->p, N, stride}, st, S, {}, kw)
             : launch_tile<128, 128, 2, 2>(W, X, N, T, K, EpiSplit{scr->p, N, stride}, st, S, {}, kw);
    if (err != hipSuccess) return err;
    if (mid && (err2 = hipEventRecord(mid, st)) != hipSuccess) return err2;
    switch (N % 1024 == 0 ? N / 1024 : 0) {
#define HB_RN(n)                                                                                \
  case n:                                                                                       \
    hipLaunchKernelGGL(splitk_reduce_norm_kernel<n>, dim3(T), dim3(256), 0, st, scr->p, S, N,   \
                       stride, e, no);                                                          \
    break;
      HB_RN(1) HB_RN(2) HB_RN(3) HB_RN(4) HB_RN(5) HB_RN(6) HB_RN(7) HB_RN(8)
#undef HB_RN
      default:
        hipLaunchKernelGGL(splitk_reduce_norm_kernel<0>, dim3(T), dim3(256), 0, st, scr->p, S, N,
                           stride, e, no);
    }
    return hipGetLastError();
  }
  const hipError_t err = launch_gemm(W, X, N, T, K, e, nullptr, st, {}, kw);
  if (err != hipSuccess) return err;
  if (mid && (err2 = hipEventRecord(mid, st)) != hipSuccess) return err2;
  return rmsnorm(e.out, N, no.gamma, T, N, no.eps, no.xn, nullptr, st, no.split);
}
hipError_t gemm_swiglu(const f16* W, const f16* X, int N, int T, int K, const EpiSwiGLU& e,
                       hipStream_t st, int kw) {
  return launch_gemm(W, X, N, T, K, e, nullptr, st, {}, kw);
}
hipError_t gemm_logits(const f16* W, const f16* X, int N, int T, int K, const EpiLogits& e,
                       hipStream_t st, int kw) {
  return launch_gemm(W, X, N, T, K, e, nullptr, st, {}, kw);
}
hipError_t gemm_qkv(const f16* W, const f16* X, int N, int T, int K, const EpiQKV& e,
                    hipStream_t st, int kw) {
  if (e.S < 1 || e.hd < 1 || e.d_pos) return hipErrorInvalidValue;  // prefill: positions from t
  auto run = [&](auto mode) {
    EpiQKVAt<false, decltype(mode)::value> ep(e);
    ep.prepare();
    return launch_gemm(W, X, N, T, K, ep, nullptr, st, {}, kw);
  };
  switch (e.mode()) {
    case EpiQKV::PLAIN: return run(std::integral_constant<int, EpiQKV::PLAIN>{});
    case EpiQKV::SPLIT: return run(std::integral_constant<int, EpiQKV::SPLIT>{});
    default: return run(std::integral_constant<int, EpiQKV::FULL>{});
  }
}


// ---- training ----
hipError_t gemm_store_split(const f16* W, const f16* X, int N, int T, int K, float* C,
                            const GemmScratch* scr, hipStream_t st, float scale) {
  return launch_gemm(W, X, N, T, K, EpiStore{C, N, scale}, scr, st);
}
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
