// Prefill GEMMs with residual epilogues (split-K, fused reduce + RMSNorm),
// the plain store, and the split counts.
#include "gemm_launch.hpp"

namespace hb {

// Split-K reduction fused with the RMSNorm that follows a residual projection
// (cpu/rmsnorm.rs:149-183): one workgroup of 256 threads per token row adds the
// splits in order, applies the residual epilogue (out = res + alpha * v), and
// normalises the row into xn. The element-to-thread mapping and the block sum
// are those of rmsnorm_kernel, so xn is bit-identical to reduce + rmsnorm.
template <int NPT, bool RAG = false>  // as rmsnorm_kernel: N = NPT * 1024 (RAG: N <= NPT * 1024) in registers, or 0 = any N
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
    auto in = [&](int i) { return !RAG || (int)threadIdx.x * 4 + i * 1024 < N; };
    f32x4 y[NPT], g[NPT];
    {
      f32x4 part[NPT][MAXS], r[NPT];
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        if (!in(i)) continue;
        const size_t c = row + threadIdx.x * 4 + i * 1024;
#pragma unroll
        for (int s = 0; s < MAXS; ++s)
          if (s < S) part[i][s] = *(const f32x4*)(P + s * stride + c);
        r[i] = *(const f32x4*)(e.res + c);
      }
#pragma unroll
      for (int i = 0; i < NPT; ++i) g[i] = in(i) ? *(const f32x4*)(no.gamma + threadIdx.x * 4 + i * 1024) : f32x4{};
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        if (!in(i)) {  // past N: adds 0 to the sum of squares
          y[i] = f32x4{};
          continue;
        }
        f32x4 v = part[i][0];
#pragma unroll
        for (int s = 1; s < MAXS; ++s)
          if (s < S) v += part[i][s];
        y[i].x = __builtin_fmaf(v.x, e.alpha, r[i].x);  // as EpiResidual
        y[i].y = __builtin_fmaf(v.y, e.alpha, r[i].y);
        y[i].z = __builtin_fmaf(v.z, e.alpha, r[i].z);
        y[i].w = __builtin_fmaf(v.w, e.alpha, r[i].w);
        *(f32x4*)(e.out + row + threadIdx.x * 4 + i * 1024) = y[i];
        ss += y[i].x * y[i].x + y[i].y * y[i].y + y[i].z * y[i].z + y[i].w * y[i].w;
      }
    }
    ss = block_sum<4>(ss, red);
    const float rinv = 1.0f / sqrtf(ss * (1.0f / (float)N) + no.eps);
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      if (!in(i)) continue;
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
      y.x = __builtin_fmaf(v.x, e.alpha, r.x);
      y.y = __builtin_fmaf(v.y, e.alpha, r.y);
      y.z = __builtin_fmaf(v.z, e.alpha, r.z);
      y.w = __builtin_fmaf(v.w, e.alpha, r.w);
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
    // 1..8: whole multiples of 1024; 9..16: ragged, ceil(N / 1024) = 1..8
    switch (N % 1024 == 0 ? N / 1024 : N % 4 == 0 && N < 8192 ? 8 + N / 1024 + 1 : 0) {
#define HB_RN(n, c, rag)                                                                        \
  case c:                                                                                       \
    hipLaunchKernelGGL((splitk_reduce_norm_kernel<n, rag>), dim3(T), dim3(256), 0, st, scr->p, S, \
                       N, stride, e, no);                                                       \
    break;
      HB_RN(1, 1, false) HB_RN(2, 2, false) HB_RN(3, 3, false) HB_RN(4, 4, false)
      HB_RN(5, 5, false) HB_RN(6, 6, false) HB_RN(7, 7, false) HB_RN(8, 8, false)
      HB_RN(1, 9, true) HB_RN(2, 10, true) HB_RN(3, 11, true) HB_RN(4, 12, true)
      HB_RN(5, 13, true) HB_RN(6, 14, true) HB_RN(7, 15, true) HB_RN(8, 16, true)
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
// ---- training ----
hipError_t gemm_store_split(const f16* W, const f16* X, int N, int T, int K, float* C,
                            const GemmScratch* scr, hipStream_t st, float scale) {
  return launch_gemm(W, X, N, T, K, EpiStore{C, N, scale}, scr, st);
}

}  // namespace hb
