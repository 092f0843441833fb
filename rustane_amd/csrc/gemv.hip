// Decode GEMV for B <= 16 sequences: y[b, n] = sum_k W[n, k] x[b, k].
//
// HBM-bound: every weight byte is read exactly once per step. The product runs
// on v_mfma_f32_16x16x32_f16 with weights as the A operand (16 rows x 32 k per
// instruction, one 16-byte load per lane = 16 rows x 64 contiguous bytes per
// wave instruction) and the B <= 16 activation rows as the B operand (columns
// >= B are zero). MFMA throughput is ~40x what the weight stream needs even at
// B = 1, and the same kernel serves every B up to 16.
//
// A workgroup owns 16*R output rows; its KS waves split K (deterministic LDS
// reduction at the end), so small-N projections (Wo, W2) still put enough
// waves in flight to saturate HBM.
#include "internal.hpp"

namespace hb {

template <int R, int KS, class Epi>
__global__ __launch_bounds__(KS * 64) void gemv_kernel(const f16* __restrict__ W,
                                                       const f16* __restrict__ X, int N, int B,
                                                       int K, Epi epi) {
  __shared__ f32x4 red[KS][R][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * 16 * R;
  const int col = lane & 15, kq = 8 * (lane >> 4);
  const int nsteps = K >> 5;
  const int s_begin = (nsteps * wave) / KS, s_end = (nsteps * (wave + 1)) / KS;

  const f16* wrow[R];
  bool rok[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = n0 + 16 * r + col;
    rok[r] = row < N;
    wrow[r] = W + (size_t)(rok[r] ? row : 0) * K + kq;
  }
  const bool xok = col < B;
  const f16* xrow = X + (size_t)(xok ? col : 0) * K + kq;

  f32x4 acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = f32x4{};
  const f16x8 zero8 = {};

  constexpr int U = 4;
  int s = s_begin;
  for (; s + U <= s_end; s += U) {
    f16x8 a[U][R], bx[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        a[u][r] = rok[r] ? *(const f16x8*)(wrow[r] + (size_t)(s + u) * 32) : zero8;
      bx[u] = xok ? *(const f16x8*)(xrow + (size_t)(s + u) * 32) : zero8;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r)
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u][r], bx[u], acc[r], 0, 0, 0);
  }
  for (; s < s_end; ++s) {
    const f16x8 bx = xok ? *(const f16x8*)(xrow + (size_t)s * 32) : zero8;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const f16x8 a = rok[r] ? *(const f16x8*)(wrow[r] + (size_t)s * 32) : zero8;
      acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bx, acc[r], 0, 0, 0);
    }
  }

#pragma unroll
  for (int r = 0; r < R; ++r) red[wave][r][lane] = acc[r];
  __syncthreads();
  if (wave == 0) {
    // acc[r][i]: row n0 + 16r + 4*(lane/16) + i, column (sequence) lane%16.
#pragma unroll
    for (int r = 0; r < R; ++r) {
      f32x4 v = red[0][r][lane];
#pragma unroll
      for (int w = 1; w < KS; ++w) v += red[w][r][lane];
      const int f0 = n0 + 16 * r + 4 * (lane >> 4);
      if (col < B && f0 < N) epi(col, f0, v);
    }
  }
}

template <class Epi>
static hipError_t launch_gemv(const f16* W, const f16* X, int N, int B, int K, const Epi& epi,
                              hipStream_t st) {
  if (B < 1 || B > 16) return hipErrorInvalidValue;
  // Aim for >= 2048 waves: few rows per workgroup and an 8-way K split when N is small.
  const int rowblocks16 = (N + 15) / 16;
  if (rowblocks16 >= 1024) {
    const int grid = (N + 31) / 32;
    hipLaunchKernelGGL((gemv_kernel<2, 4, Epi>), dim3(grid), dim3(256), 0, st, W, X, N, B, K, epi);
  } else {
    hipLaunchKernelGGL((gemv_kernel<1, 8, Epi>), dim3(rowblocks16), dim3(512), 0, st, W, X, N, B, K,
                       epi);
  }
  return hipGetLastError();
}

hipError_t gemv_residual(const f16* W, const f16* X, int N, int B, int K, const EpiResidual& e,
                         hipStream_t st) {
  return launch_gemv(W, X, N, B, K, e, st);
}
hipError_t gemv_swiglu(const f16* W, const f16* X, int N, int B, int K, const EpiSwiGLU& e,
                       hipStream_t st) {
  return launch_gemv(W, X, N, B, K, e, st);
}
hipError_t gemv_logits(const f16* W, const f16* X, int N, int B, int K, const EpiLogits& e,
                       hipStream_t st) {
  return launch_gemv(W, X, N, B, K, e, st);
}
hipError_t gemv_qkv(const f16* W, const f16* X, int N, int B, int K, const EpiQKV& e,
                    hipStream_t st) {
  return launch_gemv(W, X, N, B, K, e, st);
}
hipError_t gemv_store(const f16* W, const f16* X, int N, int B, int K, float* C, hipStream_t st) {
  return launch_gemv(W, X, N, B, K, EpiStore{C, N}, st);
}

}  // namespace hb
