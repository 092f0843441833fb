// Causal attention (kernels/sdpa_fwd.rs:132-149):
//   sc[s,t] = (Q'[s]·K'[t]) / sqrt(hd) + (t > s ? -65504 : 0); P = softmax_t(sc);
//   A[s] = sum_t P[s,t] V[t].
// The reference's additive -65504 underflows to exactly 0 after exp (every row
// keeps its diagonal term), so masked keys are skipped instead of added.
#include "internal.hpp"

namespace hb {

// ---- prefill: one wave per (32 queries, head, sequence) -------------------------
// S^T = K · Q^T on v_mfma_f32_32x32x16_f16 (rows = keys, cols = queries): lane l
// owns query l%32 and keys 8*(r/4) + 4*(l/32) + r%4 of the 32-key block, so the
// online-softmax statistics of a query live in one lane pair (l, l^32).
// O^T = V^T · P^T reuses the score registers as the B operand: with the key
// order permuted identically on both operands, lane half h supplies keys
// {16j+4h..16j+4h+3, 16j+8+4h..16j+8+4h+3} for k-step j — exactly the registers
// 8j..8j+7 it already holds — and the A operand reads those keys from V^T.
template <int HD>
__global__ __launch_bounds__(64) void attn_prefill_kernel(AttnPrefill p) {
  constexpr int KS = HD / 16;  // k-steps over head dim
  constexpr int MB = HD / 32;  // 32-row blocks of O^T
  const int lane = threadIdx.x, h2 = lane >> 5, li = lane & 31;
  const int nqb = (p.S + 31) / 32;
  const int qb = nqb - 1 - blockIdx.x;  // heaviest blocks first
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h / (p.H / p.KVH);
  const int q0 = qb * 32;
  const int qi = q0 + li;

  const f16* qp = p.q + (((size_t)b * p.H + h) * p.q_rows + q0 + li) * HD + 8 * h2;
  f16x8 qf[KS];
#pragma unroll
  for (int j = 0; j < KS; ++j) qf[j] = *(const f16x8*)(qp + 16 * j);

  const f16* kbase = p.k + b * p.k_bstride + kvh * p.k_hstride;
  const f16* vbase = p.vt + ((size_t)b * p.KVH + kvh) * HD * p.vt_ld;
  const float sl2 = p.scale * HB_LOG2E;

  f32x16 o[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) o[m] = f32x16{};
  float mrun = -INFINITY, lrun = 0.f;

  for (int kb = 0; kb <= qb; ++kb) {
    const f16* kp = kbase + (size_t)(kb * 32 + li) * HD + 8 * h2;
    f32x16 s = {};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const f16x8 kf = *(const f16x8*)(kp + 16 * j);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[j], s, 0, 0, 0);
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb * 32 + 8 * (r >> 2) + 4 * h2 + (r & 3);
      float v = s[r] * sl2;
      if (kb == qb && key > qi) v = -INFINITY;
      s[r] = v;
      mloc = fmaxf(mloc, v);
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float mnew = fmaxf(mrun, mloc);
    const float corr = exp2f(mrun - mnew);
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = exp2f(s[r] - mnew);
      s[r] = e;
      lsum += e;
    }
    lsum += __shfl_xor(lsum, 32, 64);
    lrun = lrun * corr + lsum;
    mrun = mnew;
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[m][r] *= corr;

#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f16x8 pb;
#pragma unroll
      for (int i = 0; i < 8; ++i) pb[i] = (f16)s[8 * j + i];
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const f16* vp = vbase + (size_t)(m * 32 + li) * p.vt_ld + kb * 32 + 16 * j + 4 * h2;
        const f16x4 lo = *(const f16x4*)vp;
        const f16x4 hi = *(const f16x4*)(vp + 8);
        f16x8 va;
        va[0] = lo[0]; va[1] = lo[1]; va[2] = lo[2]; va[3] = lo[3];
        va[4] = hi[0]; va[5] = hi[1]; va[6] = hi[2]; va[7] = hi[3];
        o[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o[m], 0, 0, 0);
      }
    }
  }

  if (qi < p.S) {
    const float inv = 1.0f / lrun;
    f16* op = p.out + ((size_t)b * p.S + qi) * (p.H * HD) + h * HD;
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 w;
        w.x = (f16)(o[m][4 * g + 0] * inv);
        w.y = (f16)(o[m][4 * g + 1] * inv);
        w.z = (f16)(o[m][4 * g + 2] * inv);
        w.w = (f16)(o[m][4 * g + 3] * inv);
        *(f16x4*)(op + m * 32 + 8 * g + 4 * h2) = w;
      }
  }
}

hipError_t attention_prefill(const AttnPrefill& p, hipStream_t st) {
  dim3 grid((p.S + 31) / 32, p.H, p.B);
  if (p.hd == 128)
    hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, dim3(64), 0, st, p);
  else if (p.hd == 64)
    hipLaunchKernelGGL(attn_prefill_kernel<64>, grid, dim3(64), 0, st, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// ---- decode: split the context into 256-key chunks ------------------------------
// Grid (chunk, head, sequence), 4 waves. hd/8 lanes cooperate on one key row
// (16-byte loads; a wave instruction covers 64*16 B of consecutive key rows).
// Each chunk writes its own (max, sum) and unnormalised output; a second kernel
// merges the chunks of a head. Chunks past the current position exit at once,
// so the launch shape does not depend on the position (graph-replayable).
constexpr int DCHUNK = 256;

int attn_decode_chunks(int ctx_max) { return (ctx_max + DCHUNK - 1) / DCHUNK; }

template <int HD>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecode p) {
  constexpr int LPK = HD / 8;    // lanes per key
  constexpr int KPW = 64 / LPK;  // keys per wave instruction
  constexpr int KPI = 4 * KPW;   // keys per block iteration
  __shared__ float sc[DCHUNK];
  __shared__ float red[4];
  __shared__ float oacc[4][HD];

  const int pos = *p.d_pos;
  const int c0 = blockIdx.x * DCHUNK;
  if (c0 > pos) return;
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h / (p.H / p.KVH);
  const int nch = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane / LPK, j = lane % LPK;
  const int nkeys = min(DCHUNK, pos + 1 - c0);

  const f16x8 qv = *(const f16x8*)(p.q + ((size_t)b * p.H + h) * HD + 8 * j);
  float qf[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) qf[i] = (float)qv[i];
  const f16* kb = p.k + b * p.bstride + kvh * p.hstride;
  const f16* vb = p.v + b * p.bstride + kvh * p.hstride;
  const float sl2 = p.scale * HB_LOG2E;

  for (int it = 0; it < DCHUNK; it += KPI) {
    const int kk = it + wave * KPW + g;
    float d = 0.f;
    if (kk < nkeys) {
      const f16x8 kv = *(const f16x8*)(kb + (size_t)(c0 + kk) * HD + 8 * j);
#pragma unroll
      for (int i = 0; i < 8; ++i) d += qf[i] * (float)kv[i];
    }
#pragma unroll
    for (int o = LPK / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, 64);
    if (j == 0) sc[kk] = kk < nkeys ? d * sl2 : -INFINITY;
  }
  __syncthreads();
  float m = -INFINITY;
  for (int i = tid; i < DCHUNK; i += 256) m = fmaxf(m, sc[i]);
  m = block_max<4>(m, red);
  float l = 0.f;
  for (int i = tid; i < DCHUNK; i += 256) {
    const float e = exp2f(sc[i] - m);
    sc[i] = e;
    l += e;
  }
  l = block_sum<4>(l, red);  // contains the barrier that publishes sc[]

  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int it = 0; it < DCHUNK; it += KPI) {
    const int kk = it + wave * KPW + g;
    if (kk < nkeys) {
      const float pk = sc[kk];
      const f16x8 vv = *(const f16x8*)(vb + (size_t)(c0 + kk) * HD + 8 * j);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += pk * (float)vv[i];
    }
  }
#pragma unroll
  for (int o = LPK; o < 64; o <<= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += __shfl_xor(acc[i], o, 64);
  if (g == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) oacc[wave][8 * j + i] = acc[i];
  }
  __syncthreads();
  const size_t slot = ((size_t)b * p.H + h) * nch + blockIdx.x;
  for (int e = tid; e < HD; e += 256)
    p.part_o[slot * HD + e] = oacc[0][e] + oacc[1][e] + oacc[2][e] + oacc[3][e];
  if (tid == 0) {
    p.part_ml[slot * 2] = m;
    p.part_ml[slot * 2 + 1] = l;
  }
}

template <int HD>
__global__ __launch_bounds__(HD) void attn_decode_combine_kernel(AttnDecode p, int nch) {
  const int h = blockIdx.x, b = blockIdx.y, e = threadIdx.x;
  const int pos = *p.d_pos;
  const int nvalid = pos / DCHUNK + 1;
  const size_t base = ((size_t)b * p.H + h) * nch;
  float M = -INFINITY;
  for (int c = 0; c < nvalid; ++c) M = fmaxf(M, p.part_ml[(base + c) * 2]);
  float L = 0.f, O = 0.f;
  for (int c = 0; c < nvalid; ++c) {
    const float w = exp2f(p.part_ml[(base + c) * 2] - M);
    L += w * p.part_ml[(base + c) * 2 + 1];
    O += w * p.part_o[(base + c) * HD + e];
  }
  p.out[(size_t)b * p.H * HD + h * HD + e] = (f16)(O / L);
}

hipError_t attention_decode(const AttnDecode& p, hipStream_t st) {
  const int nch = attn_decode_chunks(p.ctx_max);
  dim3 grid(nch, p.H, p.B);
  if (p.hd == 128) {
    hipLaunchKernelGGL(attn_decode_kernel<128>, grid, dim3(256), 0, st, p);
    hipLaunchKernelGGL(attn_decode_combine_kernel<128>, dim3(p.H, p.B), dim3(128), 0, st, p, nch);
  } else if (p.hd == 64) {
    hipLaunchKernelGGL(attn_decode_kernel<64>, grid, dim3(256), 0, st, p);
    hipLaunchKernelGGL(attn_decode_combine_kernel<64>, dim3(p.H, p.B), dim3(64), 0, st, p, nch);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace hb
