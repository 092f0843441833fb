// Prefill GEMM for gfx950: C^T tile = W_tile · X_tile^T on v_mfma_f32_32x32x16_f16.
//
//   W [N, K] fp16, K contiguous (weights repacked output-major at upload)
//   X [T, K] fp16, K contiguous (token-major activations)
//   result(t, f) = sum_k X[t,k] * W[f,k], fp32 accumulate, handed to an epilogue.
//
// MFMA rows are output features and MFMA columns are tokens, so each lane ends
// up holding 4 consecutive features of one token — the shape every epilogue
// (RoPE pairs, SwiGLU pairs, residual float4) wants.
//
// Pipeline per 64-wide K slice: global_load_dwordx4 of slice k+1 into registers
// is issued before the MFMAs of slice k; the registers are written to the other
// LDS buffer afterwards; one barrier per slice. LDS rows are 128 B (64 halfs) of
// eight 16-byte chunks, chunk c of row r stored at c ^ swz(r) so that both the
// ds_write_b128 of the loaders and the ds_read_b128 of the MFMA operands are
// bank-conflict free for 32- and 64-bank LDS.
#include "internal.hpp"

namespace hb {

HB_DEV int lds_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <int FT, int TT, int WF, int WT, class Epi>
__global__ __launch_bounds__(WF* WT * 64, 1) void gemm_nt_kernel(const f16* __restrict__ W,
                                                                   const f16* __restrict__ X,
                                                                   int N, int T, int K, Epi epi) {
  constexpr int NT = WF * WT * 64;
  constexpr int WFT = FT / WF, WTT = TT / WT;
  constexpr int FM = WFT / 32, TM = WTT / 32;
  constexpr int WL = FT * 8 / NT, XL = TT * 8 / NT;
  static_assert(FM >= 1 && TM >= 1, "wave tile must be at least 32x32");
  static_assert(WL * NT == FT * 8 && XL * NT == TT * 8, "loader coverage");

  __shared__ f16x8 sW[2][FT * 8];
  __shared__ f16x8 sX[2][TT * 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wf = wave / WT, wt = wave - wf * WT;
  const int nft = (N + FT - 1) / FT, ntt = (T + TT - 1) / TT;
  const int tile = xcd_remap(blockIdx.x, nft * ntt);
  const int ft = tile / ntt, tt = tile - ft * ntt;
  const int f_base = ft * FT, t_base = tt * TT;

  const f16* wsrc[WL];
  int wdst[WL];
  bool wok[WL];
#pragma unroll
  for (int i = 0; i < WL; ++i) {
    const int idx = tid + i * NT, r = idx >> 3, c = idx & 7;
    const int row = f_base + r;
    wok[i] = row < N;
    wsrc[i] = W + (size_t)(wok[i] ? row : 0) * K + c * 8;
    wdst[i] = r * 8 + (c ^ lds_swz(r));
  }
  const f16* xsrc[XL];
  int xdst[XL];
  bool xok[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int idx = tid + i * NT, r = idx >> 3, c = idx & 7;
    const int row = t_base + r;
    xok[i] = row < T;
    xsrc[i] = X + (size_t)(xok[i] ? row : 0) * K + c * 8;
    xdst[i] = r * 8 + (c ^ lds_swz(r));
  }

  f16x8 wreg[WL], xreg[XL];
  const f16x8 zero8 = {};
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < WL; ++i) wreg[i] = wok[i] ? *(const f16x8*)(wsrc[i] + k0) : zero8;
#pragma unroll
    for (int i = 0; i < XL; ++i) xreg[i] = xok[i] ? *(const f16x8*)(xsrc[i] + k0) : zero8;
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < WL; ++i) sW[buf][wdst[i]] = wreg[i];
#pragma unroll
    for (int i = 0; i < XL; ++i) sX[buf][xdst[i]] = xreg[i];
  };

  f32x16 acc[FM][TM];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x16{};

  // Fragment source rows inside the tile for this lane.
  int arow[FM], brow[TM];
#pragma unroll
  for (int i = 0; i < FM; ++i) arow[i] = wf * WFT + i * 32 + (lane & 31);
#pragma unroll
  for (int j = 0; j < TM; ++j) brow[j] = wt * WTT + j * 32 + (lane & 31);
  const int khalf = lane >> 5;

  const int nk = K / 64;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * 64);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int c = ks * 2 + khalf;
      f16x8 a[FM], b[TM];
#pragma unroll
      for (int i = 0; i < FM; ++i) a[i] = sW[cur][arow[i] * 8 + (c ^ lds_swz(arow[i]))];
#pragma unroll
      for (int j = 0; j < TM; ++j) b[j] = sX[cur][brow[j] * 8 + (c ^ lds_swz(brow[j]))];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

  // acc[i][j][r]: feature 8*(r/4) + 4*(lane/32) + r%4 of MFMA block i,
  //               token lane%32 of MFMA block j.
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) {
      const int t = t_base + wt * WTT + j * 32 + (lane & 31);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int f = f_base + wf * WFT + i * 32 + 8 * g + 4 * khalf;
        if (t < T && f < N) {
          f32x4 v;
          v.x = acc[i][j][4 * g + 0];
          v.y = acc[i][j][4 * g + 1];
          v.z = acc[i][j][4 * g + 2];
          v.w = acc[i][j][4 * g + 3];
          epi(t, f, v);
        }
      }
    }
}

template <int FT, int TT, int WF, int WT, class Epi>
static hipError_t launch_tile(const f16* W, const f16* X, int N, int T, int K, const Epi& epi,
                              hipStream_t st) {
  const int tiles = ((N + FT - 1) / FT) * ((T + TT - 1) / TT);
  hipLaunchKernelGGL((gemm_nt_kernel<FT, TT, WF, WT, Epi>), dim3(tiles), dim3(WF * WT * 64), 0,
                     st, W, X, N, T, K, epi);
  return hipGetLastError();
}

// Tile choice: the big 256x128 tile when it still yields at least one tile per
// CU, else 128x128, else 64x64 for tiny problems (decode-sized prefill, tests).
template <class Epi>
static hipError_t launch_gemm(const f16* W, const f16* X, int N, int T, int K, const Epi& epi,
                              hipStream_t st) {
  const long big = (long)((N + 255) / 256) * ((T + 127) / 128);
  const long mid = (long)((N + 127) / 128) * ((T + 127) / 128);
  if (big >= 256) return launch_tile<256, 128, 2, 2>(W, X, N, T, K, epi, st);
  if (mid >= 128) return launch_tile<128, 128, 2, 2>(W, X, N, T, K, epi, st);
  return launch_tile<64, 64, 2, 2>(W, X, N, T, K, epi, st);
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
