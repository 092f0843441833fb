// Decode GEMV for B <= 16 sequences: y[b, n] = sum_k W[n, k] x[b, k].
//
// HBM-bound: every weight byte is read exactly once per step. The product runs
// on v_mfma_f32_16x16x32_f16 with weights as the A operand (16 rows x 32 k per
// instruction) and the B <= 16 activation rows as the B operand (columns >= B
// are zero). MFMA throughput is ~40x what the weight stream needs even at
// B = 1, and the same kernel serves every B up to 16.
//
// Weights are read from a decode copy in "fragment-tiled" order: for an [N, K]
// row-major matrix, tile (rb, s) = rows 16rb..16rb+15 x columns 32s..32s+31 is
// stored as 64 consecutive 16-byte chunks, chunk `lane` holding row
// 16rb + lane%16, columns 32s + 8*(lane/16) .. +8 -- exactly lane `lane`'s A
// fragment. One wave load is one contiguous 1 KB block and a row block's whole
// K range is one contiguous run, read with nontemporal loads (the stream is
// never reused within a step, so it should not evict the activations and the
// KV cache from L2). Measured on the 7B shapes this reaches 5.5-6.5 TB/s, 20%
// above a row-major kernel of the same structure.
//
// A workgroup owns one 16-row block; its KS waves split K (deterministic LDS
// reduction at the end).
//
// Prologue RMSNorm (NORM): the projections that consume a normalised input
// (QKV, W1|W3, logits) can take the fp32 residual rows instead and normalise
// them themselves (cpu/rmsnorm.rs:149-183: r = 1/sqrt(sum(x^2)/K + eps),
// xn = x * r * gamma, rounded to fp16). Every workgroup reads whole rows of x
// anyway, so each computes the sums of squares of the B rows itself, stages xn
// in LDS and takes its B operand from there. The first weight loads are issued
// before the prologue, so the x reads overlap the HBM latency. This removes a
// launch per norm without putting any extra memory round trip on the critical
// path; it is used while the B staged rows fit in GEMV_NORM_LDS bytes.
//
// Attention prologue (Wo only): the decode attention leaves one partial
// (max, sum, unnormalised output) per chunk of the context, and every Wo
// workgroup merges them into the fp16 attention rows it needs (all of them)
// in the same way. With B * chunks <= GEMV_ATTN_MAXCH that is at most
// 8 x 130 floats per (sequence, head) -- 133 KB per workgroup on the 7B shape --
// fetched while the first weight loads are in flight, instead of a separate
// combine launch (attention_combine, used when B * chunks is larger).
#include <type_traits>

#include "internal.hpp"

namespace hb {

__global__ __launch_bounds__(256) void tile_decode_kernel(const f16* __restrict__ W,
                                                          f16x8* __restrict__ Wt, int N, int K) {
  const int nks = K >> 5;
  const size_t total = (size_t)(N >> 4) * nks * 64;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const int lane = (int)(i & 63);
    const size_t t = i >> 6;
    const int s = (int)(t % nks);
    const size_t rb = t / nks;
    Wt[i] = *(const f16x8*)(W + (rb * 16 + (lane & 15)) * (size_t)K + s * 32 + 8 * (lane >> 4));
  }
}

hipError_t tile_decode(const f16* W, f16* Wt, int N, int K, hipStream_t st) {
  if (N % 16 || K % 32) return hipErrorInvalidValue;
  const size_t chunks = (size_t)N * K / 8;
  const int grid = (int)std::min<size_t>((chunks + 255) / 256, 8192);
  hipLaunchKernelGGL(tile_decode_kernel, dim3(grid), dim3(256), 0, st, W, (f16x8*)Wt, N, K);
  return hipGetLastError();
}

// Row stride (in halves) of the staged xn rows: +8 halves keeps the B <= 4
// rows of one ds_read_b128 on different banks.
HB_DEV int xn_ld(int K) { return K + 8; }

// xn[b][k] = fp16(x[b][k] * r_b * gamma[k]) for b < B into LDS, by all NT
// threads of the workgroup. K % 8 == 0.
template <int NT>
HB_DEV void stage_norm(const NormIn& nin, int B, int K, f16* s_x) {
  constexpr int NW = NT / 64;
  __shared__ float s_part[NW][GEMV_NORM_MAXB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float ss[GEMV_NORM_MAXB];
#pragma unroll
  for (int b = 0; b < GEMV_NORM_MAXB; ++b) {
    ss[b] = 0.f;
    if (b < B) {
      const float* xr = nin.x + (size_t)b * K;
      for (int c = tid * 8; c < K; c += NT * 8) {
        const f32x4 u = *(const f32x4*)(xr + c), v = *(const f32x4*)(xr + c + 4);
        ss[b] += u.x * u.x + u.y * u.y + u.z * u.z + u.w * u.w + v.x * v.x + v.y * v.y +
                 v.z * v.z + v.w * v.w;
      }
    }
    ss[b] = wave_sum(ss[b]);
    if (lane == 0) s_part[wave][b] = ss[b];
  }
  __syncthreads();
  const int ld = xn_ld(K);
  for (int b = 0; b < B; ++b) {
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += s_part[w][b];
    const float r = 1.0f / sqrtf(tot * (1.0f / (float)K) + nin.eps);
    const float* xr = nin.x + (size_t)b * K;
    for (int c = tid * 8; c < K; c += NT * 8) {
      const f32x4 u = *(const f32x4*)(xr + c), v = *(const f32x4*)(xr + c + 4);
      const f32x4 g = *(const f32x4*)(nin.gamma + c), h = *(const f32x4*)(nin.gamma + c + 4);
      f16x8 o;
      o[0] = (f16)(u.x * r * g.x);
      o[1] = (f16)(u.y * r * g.y);
      o[2] = (f16)(u.z * r * g.z);
      o[3] = (f16)(u.w * r * g.w);
      o[4] = (f16)(v.x * r * h.x);
      o[5] = (f16)(v.y * r * h.y);
      o[6] = (f16)(v.z * r * h.z);
      o[7] = (f16)(v.w * r * h.w);
      *(f16x8*)(s_x + b * ld + c) = o;
    }
  }
  __syncthreads();
}

// attn[b][h*hd + e] = fp16(sum_c w_c o_c[e] / sum_c w_c l_c), w_c = exp2(m_c - M),
// M = max_c m_c over the chunks of attention_decode that hold keys -- the
// arithmetic and chunk order of attention_combine. One 8-dim group of one
// (sequence, head) per thread and pass: the chunk maxima first, then the
// chunk outputs in batches of 8 with every load of a batch issued before any
// is used.
template <int NT>
HB_DEV void stage_attn(const AttnIn& ai, int B, int K, f16* s_x) {
  constexpr int MAXCH = GEMV_ATTN_MAXCH;
  constexpr int CB = 8;  // chunk outputs in flight per batch
  const int nvalid = attn_chunks_valid(*ai.d_pos, ai.nch);
  const int gph = ai.hd / 8;
  const int ngroups = B * ai.H * gph;
  const int ld = xn_ld(K);
  for (int gi = threadIdx.x; gi < ngroups; gi += NT) {
    const int e0 = (gi % gph) * 8;
    const int bh = gi / gph;  // b * H + h
    const int b = bh / ai.H, h = bh - b * ai.H;
    const float* pml = ai.part_ml + (size_t)bh * ai.nch * 2;
    const float* po = ai.part_o + (size_t)bh * ai.nch * ai.hd + e0;
    float m[MAXCH];
#pragma unroll
    for (int c = 0; c < MAXCH; ++c)
      if (c < nvalid) m[c] = pml[2 * c];
    float M = -INFINITY;
#pragma unroll
    for (int c = 0; c < MAXCH; ++c)
      if (c < nvalid) M = fmaxf(M, m[c]);
    float L = 0.f;
    f32x4 O0 = {}, O1 = {};
#pragma unroll
    for (int cb = 0; cb < MAXCH; cb += CB) {
      float l[CB];
      f32x4 u[CB], v[CB];
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const int c = cb + j;
        if (c < nvalid) {
          l[j] = pml[2 * c + 1];
          u[j] = *(const f32x4*)(po + (size_t)c * ai.hd);
          v[j] = *(const f32x4*)(po + (size_t)c * ai.hd + 4);
        }
      }
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const int c = cb + j;
        if (c < nvalid) {
          const float w = exp2f(m[c] - M);
          L += w * l[j];
          O0 += w * u[j];
          O1 += w * v[j];
        }
      }
    }
    const float iL = 1.0f / L;
    f16x8 o;
    o[0] = (f16)(O0.x * iL);
    o[1] = (f16)(O0.y * iL);
    o[2] = (f16)(O0.z * iL);
    o[3] = (f16)(O0.w * iL);
    o[4] = (f16)(O1.x * iL);
    o[5] = (f16)(O1.y * iL);
    o[6] = (f16)(O1.z * iL);
    o[7] = (f16)(O1.w * iL);
    *(f16x8*)(s_x + b * ld + h * ai.hd + e0) = o;
  }
  __syncthreads();
}

// Greedy-decode argmax partials of the logits epilogue: the first index of
// the maximum of each sequence's 16 logits of this row block (NaN never
// wins, ties go to the lower index).
HB_DEV void argmax_partial(const EpiLogits& e, f32x4 v, int f0, int col, int B, int rb, int nrb) {
  const f32x4 y = e.capped(v);
  float best = -INFINITY;
  int idx = 0x7fffffff;
  if (y.x > best) { best = y.x; idx = f0; }
  if (y.y > best) { best = y.y; idx = f0 + 1; }
  if (y.z > best) { best = y.z; idx = f0 + 2; }
  if (y.w > best) { best = y.w; idx = f0 + 3; }
#pragma unroll
  for (int o = 16; o < 64; o <<= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (ob > best || (ob == best && oi < idx)) {
      best = ob;
      idx = oi;
    }
  }
  if ((threadIdx.x & 63) < 16 && col < B) {
    const size_t slot = (size_t)col * nrb + rb;
    e.part_val[slot] = best;
    e.part_idx[slot] = idx;
  }
}

// Prologue kinds: the B operand comes from X (PRO_NONE) or from rows staged
// in LDS by stage_norm (PRO_NORM) or stage_attn (PRO_ATTN).
enum { PRO_NONE = 0, PRO_NORM = 1, PRO_ATTN = 2 };

// SPLIT (PRO_NONE only): X rows are split rows [B][2K] (common.hpp); every
// weight fragment meets the hi and the lo half of the B operand, two MFMAs
// into the same accumulator, so the weight stream is read once.
// XFRAG (PRO_NONE only): X is in B-fragment order (EpiSwiGLU::frag): the
// operand of k-step s is the 1 KB block X + s*512, lane l's 16 bytes at l*8.
template <int KS, int U, class Epi, int PRO, bool SPLIT, bool XFRAG = false>
__global__ __launch_bounds__(KS * 64) void gemv_kernel(const f16x8* __restrict__ Wt,
                                                       const f16* __restrict__ X, int N, int B,
                                                       int K, Epi epi, NormIn nin, AttnIn ain) {
  static_assert(!SPLIT || PRO == PRO_NONE, "split rows come from memory");
  static_assert(!XFRAG || (PRO == PRO_NONE && !SPLIT), "fragment-order rows come from memory");
  extern __shared__ f16x8 s_dyn[];  // staged B-operand rows [B][xn_ld(K)]
  __shared__ f32x4 red[KS][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rb = blockIdx.x;
  const int col = lane & 15, kq = 8 * (lane >> 4);
  const int nsteps = K >> 5;
  const int s_begin = (nsteps * wave) / KS, s_end = (nsteps * (wave + 1)) / KS;
  const f16x8* wp = Wt + (size_t)rb * nsteps * 64 + lane;
  const bool xok = col < B;
  const f16* s_x = (const f16*)s_dyn;
  const f16* xrow = PRO != PRO_NONE ? s_x + (xok ? col : 0) * xn_ld(K) + kq
                                     : X + (size_t)(xok ? col : 0) * (SPLIT ? 2 * K : K) + kq;
  auto bop = [&](int s) -> f16x8 {
    const f16x8 zero8 = {};
    if constexpr (XFRAG) return xok ? *(const f16x8*)(X + ((size_t)s * 64 + lane) * 8) : zero8;
    return xok ? *(const f16x8*)(xrow + (size_t)s * 32) : zero8;
  };
  auto bopl = [&](int s) -> f16x8 {  // low half of a split row
    const f16x8 zero8 = {};
    return xok ? *(const f16x8*)(xrow + K + (size_t)s * 32) : zero8;
  };

  f32x4 acc = {};
  int s = s_begin;
  if constexpr (PRO != PRO_NONE) {
    // Keep the weight stream busy through the prologue: up to PF fragments
    // per wave are in flight before it starts. Wo (attention prologue) runs
    // one workgroup per CU, so it can hold its whole 7B slice (16 steps).
    constexpr int PF = PRO == PRO_ATTN ? 16 : 8;
    f16x8 a[PF];
    const int npf = min(PF, s_end - s);
#pragma unroll
    for (int u = 0; u < PF; ++u)
      if (u < npf) a[u] = __builtin_nontemporal_load(wp + (size_t)(s + u) * 64);
    if constexpr (PRO == PRO_NORM)
      stage_norm<KS * 64>(nin, B, K, (f16*)s_dyn);
    else
      stage_attn<KS * 64>(ain, B, K, (f16*)s_dyn);
#pragma unroll
    for (int u = 0; u < PF; ++u)
      if (u < npf) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], bop(s + u), acc, 0, 0, 0);
    s += npf;
  }
  for (; s + U <= s_end; s += U) {
    f16x8 a[U], bx[U], bl[SPLIT ? U : 1];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      a[u] = __builtin_nontemporal_load(wp + (size_t)(s + u) * 64);
      bx[u] = bop(s + u);
      if constexpr (SPLIT) bl[u] = bopl(s + u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], bx[u], acc, 0, 0, 0);
      if constexpr (SPLIT) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], bl[u], acc, 0, 0, 0);
    }
  }
  for (; s < s_end; ++s) {
    const f16x8 a = __builtin_nontemporal_load(wp + (size_t)s * 64);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bop(s), acc, 0, 0, 0);
    if constexpr (SPLIT) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bopl(s), acc, 0, 0, 0);
  }

  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0) {
    // acc[i]: row 16rb + 4*(lane/16) + i, column (sequence) lane%16.
    f32x4 v = red[0][lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) v += red[w][lane];
    const int f0 = rb * 16 + 4 * (lane >> 4);
    if (col < B) epi(col, f0, v);
    if constexpr (std::is_same_v<Epi, EpiLogits>) {
      if (epi.part_val) argmax_partial(epi, v, f0, col, B, rb, gridDim.x);
    }
  }
}

// Wide batches (B > 3, no norm prologue): every lane of a wave reads the B
// operand, as many bytes per k-step as the weight fragment, and the plain
// kernel re-reads all B rows for each 16-row block. Here a workgroup walks R
// row blocks (blockIdx.x, + gridDim.x, ...) and each wave keeps its K range of
// the B rows in registers (XS fragments, K <= 32 * XS * KS), so the rows are
// read once per workgroup. Same per-block arithmetic as gemv_kernel (one
// MFMA chain per wave over its K range, waves summed in order).
template <int KS, int XS, int U, class Epi, bool XFRAG = false>
__global__ __launch_bounds__(KS * 64) void gemv_xreg_kernel(const f16x8* __restrict__ Wt,
                                                            const f16* __restrict__ X, int N, int B,
                                                            int K, Epi epi) {
  __shared__ f32x4 red[KS][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, kq = 8 * (lane >> 4);
  const int nsteps = K >> 5;
  const int s_begin = (nsteps * wave) / KS, ns = (nsteps * (wave + 1)) / KS - s_begin;  // ns <= XS
  const bool xok = col < B;
  const f16* xrow = X + (size_t)(xok ? col : 0) * K + kq + (size_t)s_begin * 32;
  const f16x8 zero8 = {};
  f16x8 xr[XS];
#pragma unroll
  for (int j = 0; j < XS; ++j) {
    f16x8 v = zero8;
    if (j < ns) {
      if constexpr (XFRAG)  // B-fragment order: k-step s at X + s*512
        v = *(const f16x8*)(X + ((size_t)(s_begin + j) * 64 + lane) * 8);
      else
        v = *(const f16x8*)(xrow + (size_t)j * 32);
    }
    xr[j] = xok ? v : zero8;
  }
  const int nrb = N >> 4;
  for (int rb = blockIdx.x; rb < nrb; rb += gridDim.x) {
    const f16x8* wp = Wt + ((size_t)rb * nsteps + s_begin) * 64 + lane;
    f32x4 acc = {};
#pragma unroll
    for (int j0 = 0; j0 < XS; j0 += U) {
      f16x8 a[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (j0 + u < ns) a[u] = __builtin_nontemporal_load(wp + (size_t)(j0 + u) * 64);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (j0 + u < ns) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], xr[j0 + u], acc, 0, 0, 0);
    }
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
      f32x4 v = red[0][lane];
#pragma unroll
      for (int w = 1; w < KS; ++w) v += red[w][lane];
      const int f0 = rb * 16 + 4 * (lane >> 4);
      if (col < B) epi(col, f0, v);
      if constexpr (std::is_same_v<Epi, EpiLogits>) {
        if (epi.part_val) argmax_partial(epi, v, f0, col, B, rb, nrb);
      }
    }
    __syncthreads();  // red is reused by the next row block
  }
}

namespace {
constexpr int GEMV_KS = 8;  // waves per workgroup (K split)
// gemv_xreg_kernel: B-operand fragments per wave (K <= 4096), batches from
// which it is used, workgroups (one per CU: 7B at B = 16, 6.78 -> 6.56 ms per
// decode step; two per CU and half the row blocks each: 6.76) and weight
// loads in flight per wave (4: 6.60 ms, 16: 7.18)
constexpr int GEMV_XS = 16;
constexpr int GEMV_XREG_MINB = 4;
constexpr int GEMV_XREG_WGS = 256;
constexpr int GEMV_XREG_U = 8;
constexpr int GEMV_U = 4;   // 1 KB weight loads in flight per wave

template <class Epi>
hipError_t launch_gemv(const f16* Wt, const f16* X, const NormIn* nin, const AttnIn* ain, int N,
                       int B, int K, const Epi& epi, hipStream_t st, bool split = false,
                       bool xfrag = false) {
  if (B < 1 || B > 16 || N % 16 || K % 32) return hipErrorInvalidValue;
  if (xfrag) {  // X in B-fragment order (no prologue)
    if (split || nin || ain) return hipErrorInvalidValue;
    if (K <= 32 * GEMV_XS * GEMV_KS && N / 16 > GEMV_XREG_WGS) {
      const int nrb = N / 16, per = (nrb + GEMV_XREG_WGS - 1) / GEMV_XREG_WGS;
      hipLaunchKernelGGL((gemv_xreg_kernel<GEMV_KS, GEMV_XS, GEMV_XREG_U, Epi, true>), dim3((nrb + per - 1) / per),
                         dim3(GEMV_KS * 64), 0, st, (const f16x8*)Wt, X, N, B, K, epi);
    } else {
      hipLaunchKernelGGL((gemv_kernel<GEMV_KS, GEMV_U, Epi, PRO_NONE, false, true>), dim3(N / 16),
                         dim3(GEMV_KS * 64), 0, st, (const f16x8*)Wt, X, N, B, K, epi, NormIn{},
                         AttnIn{});
    }
    return hipGetLastError();
  }
  if (split) {
    if (nin || ain) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_kernel<GEMV_KS, GEMV_U, Epi, PRO_NONE, true>), dim3(N / 16),
                       dim3(GEMV_KS * 64), 0, st, (const f16x8*)Wt, X, N, B, K, epi, NormIn{},
                       AttnIn{});
    return hipGetLastError();
  }
  const dim3 grid(N / 16), block(GEMV_KS * 64);
  const size_t lds = (size_t)B * (K + 8) * 2;
  // Only the projections fed by a norm (QKV, W1|W3, logits) have a norm
  // prologue, and only Wo (residual epilogue) the attention combine.
  constexpr bool kNorm = !std::is_same_v<Epi, EpiResidual> && !std::is_same_v<Epi, EpiStore>;
  constexpr bool kAttn = std::is_same_v<Epi, EpiResidual>;
  if (nin) {
    if constexpr (kNorm) {
      if (!gemv_norm_fits(B, K)) return hipErrorInvalidValue;
      hipLaunchKernelGGL((gemv_kernel<GEMV_KS, GEMV_U, Epi, PRO_NORM, false>), grid, block, lds, st,
                         (const f16x8*)Wt, nullptr, N, B, K, epi, *nin, AttnIn{});
    } else {
      return hipErrorInvalidValue;
    }
  } else if (ain) {
    if constexpr (kAttn) {
      if (!gemv_attn_fits(B, K, ain->nch) || ain->H * ain->hd != K || ain->hd % 8) return hipErrorInvalidValue;
      hipLaunchKernelGGL((gemv_kernel<GEMV_KS, GEMV_U, Epi, PRO_ATTN, false>), grid, block, lds, st,
                         (const f16x8*)Wt, nullptr, N, B, K, epi, NormIn{}, *ain);
    } else {
      return hipErrorInvalidValue;
    }
  } else if (B >= GEMV_XREG_MINB && K <= 32 * GEMV_XS * GEMV_KS && N / 16 > GEMV_XREG_WGS) {
    // several row blocks per workgroup: at most GEMV_XREG_WGS workgroups
    const int nrb = N / 16, per = (nrb + GEMV_XREG_WGS - 1) / GEMV_XREG_WGS;
    hipLaunchKernelGGL((gemv_xreg_kernel<GEMV_KS, GEMV_XS, GEMV_XREG_U, Epi>), dim3((nrb + per - 1) / per), block, 0,
                       st, (const f16x8*)Wt, X, N, B, K, epi);
  } else {
    hipLaunchKernelGGL((gemv_kernel<GEMV_KS, GEMV_U, Epi, PRO_NONE, false>), grid, block, 0, st,
                       (const f16x8*)Wt, X, N, B, K, epi, NormIn{}, AttnIn{});
  }
  return hipGetLastError();
}
}  // namespace

bool gemv_norm_fits(int B, int K) {
  return B >= 1 && B <= GEMV_NORM_MAXB && (size_t)B * (K + 8) * 2 <= GEMV_NORM_LDS;
}
bool gemv_attn_fits(int B, int K, int nch) {
  return B >= 1 && nch >= 1 && B * nch <= GEMV_ATTN_MAXCH &&
         (size_t)B * (K + 8) * 2 <= GEMV_NORM_LDS;
}

hipError_t gemv_residual(const f16* Wt, const f16* X, const AttnIn* ain, int N, int B, int K,
                         const EpiResidual& e, hipStream_t st, bool split, bool xfrag) {
  return launch_gemv(Wt, X, nullptr, ain, N, B, K, e, st, split, xfrag);
}
hipError_t gemv_swiglu(const f16* Wt, const f16* X, const NormIn* nin, int N, int B, int K,
                       const EpiSwiGLU& e, hipStream_t st, bool split, bool xfrag) {
  if (e.frag) {
    if (e.split || e.tap || B > 16 || e.hidden % 32) return hipErrorInvalidValue;
    return launch_gemv(Wt, X, nin, nullptr, N, B, K, EpiSwiGLUFrag{e.gate}, st, split, xfrag);
  }
  return launch_gemv(Wt, X, nin, nullptr, N, B, K, e, st, split, xfrag);
}
hipError_t gemv_logits(const f16* Wt, const f16* X, const NormIn* nin, int N, int B, int K,
                       const EpiLogits& e, hipStream_t st, bool split, bool xfrag) {
  return launch_gemv(Wt, X, nin, nullptr, N, B, K, e, st, split, xfrag);
}
hipError_t gemv_qkv(const f16* Wt, const f16* X, const NormIn* nin, int N, int B, int K,
                    const EpiQKV& e, hipStream_t st, bool split, bool xfrag) {
  if (e.S < 1 || e.hd < 1) return hipErrorInvalidValue;
  auto run = [&](auto dec, auto mode) {
    EpiQKVAt<decltype(dec)::value, decltype(mode)::value> ep(e);
    ep.prepare();
    return launch_gemv(Wt, X, nin, nullptr, N, B, K, ep, st, split, xfrag);
  };
  using Dec = std::integral_constant<bool, true>;
  using Pre = std::integral_constant<bool, false>;
  using Plain = std::integral_constant<int, EpiQKV::PLAIN>;
  using Split = std::integral_constant<int, EpiQKV::SPLIT>;
  using Full = std::integral_constant<int, EpiQKV::FULL>;
  const int mode = e.mode();
  if (e.d_pos)
    return mode == EpiQKV::PLAIN ? run(Dec{}, Plain{}) : mode == EpiQKV::SPLIT ? run(Dec{}, Split{}) : run(Dec{}, Full{});
  return mode == EpiQKV::PLAIN ? run(Pre{}, Plain{}) : mode == EpiQKV::SPLIT ? run(Pre{}, Split{}) : run(Pre{}, Full{});
}
hipError_t gemv_store(const f16* Wt, const f16* X, int N, int B, int K, float* C, hipStream_t st) {
  return launch_gemv(Wt, X, nullptr, nullptr, N, B, K, EpiStore{C, N}, st);
}

// ---- greedy token: reduce the argmax partials, advance the decode state ----
// One workgroup per call (4 waves for B <= 4, else 16), NW / B waves (at
// least one) per sequence, all sequences at once: each wave folds a strided
// share of its sequence's partials (8 loads in flight per batch), then the
// sequence's waves reduce through LDS, with the same rules as argmax_partial
// (the result is the first index of the maximum whatever the folding order). With
// tok/d_pos set it also does the decode-step bookkeeping: the token becomes
// the next step's input, is appended to the history at row (pos - pos0), and
// the position advances.
HB_DEV void amax_fold(float& best, int& idx, float v, int j) {
  if (v > best || (v == best && j < idx)) {
    best = v;
    idx = j;
  }
}

template <int NW>
__global__ __launch_bounds__(NW * 64) void argmax_reduce_kernel(
    const float* __restrict__ pval, const int* __restrict__ pidx, int nblk, int B,
    uint32_t* __restrict__ next, uint32_t* tok, uint32_t* hist, int* d_pos, const int* d_pos0) {
  constexpr int NB = 8;
  __shared__ float s_v[NW];
  __shared__ int s_i[NW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wps = max(1, NW / B);  // waves per sequence
  const int b = wave / wps, r = wave - b * wps;
  const int pos = d_pos ? *d_pos : 0;
  float best = -INFINITY;
  int idx = 0x7fffffff;
  if (b < B) {
    const float* pv = pval + (size_t)b * nblk;
    const int* pi = pidx + (size_t)b * nblk;
    const int stride = wps * 64;
    for (int i0 = r * 64 + lane; i0 < nblk; i0 += stride * NB) {
      float v[NB];
      int j[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int i = i0 + u * stride;
        v[u] = i < nblk ? pv[i] : -INFINITY;
        j[u] = i < nblk ? pi[i] : 0x7fffffff;
      }
#pragma unroll
      for (int u = 0; u < NB; ++u) amax_fold(best, idx, v[u], j[u]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) amax_fold(best, idx, __shfl_xor(best, o, 64), __shfl_xor(idx, o, 64));
  }
  if (lane == 0) {
    s_v[wave] = best;
    s_i[wave] = idx;
  }
  __syncthreads();  // also: every thread has read *d_pos
  if (b < B && r == 0 && lane == 0) {
    for (int w = 1; w < wps; ++w) amax_fold(best, idx, s_v[wave + w], s_i[wave + w]);
    next[b] = (uint32_t)idx;
    if (tok) {
      tok[b] = (uint32_t)idx;
      if (hist) hist[(size_t)(pos - *d_pos0) * B + b] = (uint32_t)idx;
    }
  }
  if (d_pos && tid == 0) *d_pos = pos + 1;
}

hipError_t argmax_reduce(const float* pval, const int* pidx, int nblk, int B, uint32_t* next,
                         uint32_t* tok, uint32_t* hist, int* d_pos, const int* d_pos0,
                         hipStream_t st) {
  if (B < 1 || B > 16 || nblk < 1) return hipErrorInvalidValue;
  // 4 waves fold one sequence's 2000 partials (7B vocab) in one batch of
  // loads; wide batches take a wave per sequence (B = 16: 31 -> 7.7 us)
  if (B <= 4)
    hipLaunchKernelGGL(argmax_reduce_kernel<4>, dim3(1), dim3(256), 0, st, pval, pidx, nblk, B, next, tok, hist,
                       d_pos, d_pos0);
  else
    hipLaunchKernelGGL(argmax_reduce_kernel<16>, dim3(1), dim3(1024), 0, st, pval, pidx, nblk, B, next, tok, hist,
                       d_pos, d_pos0);
  return hipGetLastError();
}

}  // namespace hb
