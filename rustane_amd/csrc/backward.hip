// Training backward: the elementwise and reduction kernels between the
// backward GEMMs (gemm_train.hip, epilogues in epilogue.hpp). Everything here is
// HBM-bound byte work; the products themselves run on the MFMA GEMM.
//
// Layout conventions of the backward (the reference works channel-first
// [dim, seq] with CPU sgemms for dW, layer.rs:1606-1858; this build keeps
// activations token-major [T, features] like its forward):
//   dX products   C[T, N] = dY[T, K] · W^T       read transposed fp16 weights
//   dW products   dW[n, k] += sum_t A[t, n] B[t, k] read feature-major copies
//                 [features][Tp] of both activations (Tp = T rounded up to 64,
//                 padding columns zero) so that the token sum is the GEMM's K.
#include "internal.hpp"

namespace hb {

// ---- transposes ------------------------------------------------------------
// dst[b][c][r] = scale * src[b][r][c] as fp16 for r < R, c < C; dst columns
// r in [R, ldd) are written as zero. With rm != NULL (batch 1) the scaled fp16
// values are also stored row-major: rm[r * C + c]. 64x64 tiles through LDS:
// loads coalesced along c, stores along r.
template <class S>
__global__ __launch_bounds__(256) void transpose_kernel(const S* __restrict__ src, int R, int C,
                                                        int lds, size_t sbs, float scale,
                                                        f16* __restrict__ dst, int ldd, size_t dbs,
                                                        f16* __restrict__ rm) {
  __shared__ float tile[64][65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  src += blockIdx.z * sbs;
  dst += blockIdx.z * dbs;
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int r = r0 + ty + 4 * i, c = c0 + tx;
    float v = 0.f;
    if (r < R && c < C) {
      v = (float)src[(size_t)r * lds + c] * scale;
      if (rm) rm[(size_t)r * C + c] = (f16)v;
    }
    tile[ty + 4 * i][tx] = v;
  }
  __syncthreads();
#pragma unroll 4
  for (int i = 0; i < 16; ++i) {
    const int c = c0 + ty + 4 * i, r = r0 + tx;
    if (c < C && r < ldd) dst[(size_t)c * ldd + r] = (f16)tile[tx][ty + 4 * i];
  }
}

// fp16 -> fp16 with 16-byte global accesses when C, lds, ldd, the batch
// strides and both pointers are multiples of 8 halfs: 64x64 tiles, each
// thread loads two 8-half row chunks and stores two 8-half column chunks
// gathered from LDS (row pitch 72 halfs keeps the 16-byte LDS writes aligned).
__global__ __launch_bounds__(256) void transpose16_kernel(const f16* __restrict__ src, int R, int C,
                                                          int lds, size_t sbs,
                                                          f16* __restrict__ dst, int ldd,
                                                          size_t dbs) {
  __shared__ f16x8 tile[64 * 9];  // [64 rows][72 halfs]
  const int tid = threadIdx.x, c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  src += blockIdx.z * sbs;
  dst += blockIdx.z * dbs;
  const int lr = tid >> 3, lc = (tid & 7) * 8;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int r = r0 + p * 32 + lr, c = c0 + lc;
    f16x8 v = {};
    if (r < R && c < C) v = *(const f16x8*)(src + (size_t)r * lds + c);
    tile[(p * 32 + lr) * 9 + (lc >> 3)] = v;
  }
  __syncthreads();
  const f16* t = (const f16*)tile;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int c = p * 32 + lr, rr = lc;
    f16x8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = t[(rr + j) * 72 + c];
    if (c0 + c < C && r0 + rr < ldd) *(f16x8*)(dst + (size_t)(c0 + c) * ldd + r0 + rr) = h;
  }
}

hipError_t transpose_f16(const f16* src, int R, int C, int lds, size_t sbs, f16* dst, int ldd,
                         size_t dbs, int batch, hipStream_t st) {
  if (R < 0 || C < 0 || ldd < R || lds < C || batch < 1 || batch > 65535) return hipErrorInvalidValue;
  if (C == 0 || ldd == 0) return hipSuccess;
  const bool v16 = C % 8 == 0 && lds % 8 == 0 && ldd % 8 == 0 && sbs % 8 == 0 && dbs % 8 == 0 &&
                   ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0;
  if (v16) {
    hipLaunchKernelGGL(transpose16_kernel, dim3((C + 63) / 64, (ldd + 63) / 64, batch), dim3(256), 0,
                       st, src, R, C, lds, sbs, dst, ldd, dbs);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(transpose_kernel<f16>, dim3((C + 63) / 64, (ldd + 63) / 64, batch), dim3(256), 0,
                     st, src, R, C, lds, sbs, 1.0f, dst, ldd, dbs, (f16*)nullptr);
  return hipGetLastError();
}

hipError_t cast_transpose(const float* src, int R, int C, float scale, f16* rm, f16* dst, int ldd,
                          hipStream_t st) {
  if (R < 0 || C < 0 || ldd < R) return hipErrorInvalidValue;
  if (C == 0 || ldd == 0) return hipSuccess;
  hipLaunchKernelGGL(transpose_kernel<float>, dim3((C + 63) / 64, (ldd + 63) / 64, 1), dim3(256), 0,
                     st, src, R, C, C, (size_t)0, scale, dst, ldd, (size_t)0, rm);
  return hipGetLastError();
}

// ---- cross-entropy backward ---------------------------------------------------
// One workgroup per position t (full_model.rs:242-246 and 265-276 with
// cpu/cross_entropy.rs:58-96): p = softmax(z) over the (capped) logits,
// dl = (p - onehot(y)) * gs with gs = loss_scale / S, times (1 - tc^2) with
// tc = z / softcap when the logits went through softcap * tanh(. / softcap).
// Written as fp16 [T][Vp], columns [V, Vp) zero.
__global__ __launch_bounds__(256) void ce_backward_kernel(const float* __restrict__ logits,
                                                          const uint32_t* __restrict__ tgt, int V,
                                                          int Vp, float gs, float softcap,
                                                          f16* __restrict__ dl) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const float* z = logits + (size_t)t * V;
  float m = -INFINITY;
  for (int v = threadIdx.x; v < V; v += 256) m = fmaxf(m, z[v]);
  m = block_max<4>(m, red);
  float se = 0.f;
  for (int v = threadIdx.x; v < V; v += 256) se += expf(z[v] - m);
  se = block_sum<4>(se, red);
  const float inv = 1.0f / se;
  const uint32_t y = tgt[t];
  const float ic = softcap > 0.f ? 1.0f / softcap : 0.f;
  f16* o = dl + (size_t)t * Vp;
  for (int v = threadIdx.x; v < Vp; v += 256) {
    float d = 0.f;
    if (v < V) {
      const float zv = z[v];
      d = expf(zv - m) * inv - ((uint32_t)v == y ? 1.0f : 0.0f);
      d *= gs;
      if (softcap > 0.f) {
        const float tc = zv * ic;
        d *= 1.0f - tc * tc;
      }
    }
    o[v] = (f16)d;
  }
}

hipError_t ce_backward(const float* logits, const uint32_t* tgt, int T, int V, int Vp, float gs,
                       float softcap, f16* dl, hipStream_t st) {
  if (T < 0 || V < 1 || Vp < V) return hipErrorInvalidValue;
  if (T == 0) return hipSuccess;
  hipLaunchKernelGGL(ce_backward_kernel, dim3(T), dim3(256), 0, st, logits, tgt, V, Vp, gs, softcap,
                     dl);
  return hipGetLastError();
}

// ---- ForwardResult views (full_model.rs:73-81) -------------------------------------
// dlogits as forward() returns them (cpu/cross_entropy.rs:58-96, scaled by
// 1/seq): e = exp(z - max), d = e * (1/sum e), d[y] -= 1, d *= inv_seq; and
// logits_capped = tanh(raw / softcap) (full_model.rs:388-393), recovered from
// the stored capped logits z = softcap * t as z * (1/softcap). fp32 [T][V].
__global__ __launch_bounds__(256) void ce_grad_views_kernel(const float* __restrict__ logits,
                                                            const uint32_t* __restrict__ tgt, int V,
                                                            float inv_seq, float softcap,
                                                            float* __restrict__ dl,
                                                            float* __restrict__ tcap) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const float* z = logits + (size_t)t * V;
  float m = -INFINITY;
  for (int v = threadIdx.x; v < V; v += 256) m = fmaxf(m, z[v]);
  m = block_max<4>(m, red);
  float se = 0.f;
  for (int v = threadIdx.x; v < V; v += 256) se += expf(z[v] - m);
  se = block_sum<4>(se, red);
  const float inv = 1.0f / se, ic = softcap > 0.f ? 1.0f / softcap : 0.f;
  const uint32_t y = tgt[t];
  for (int v = threadIdx.x; v < V; v += 256) {
    const float zv = z[v];
    if (dl) dl[(size_t)t * V + v] = (expf(zv - m) * inv - ((uint32_t)v == y ? 1.0f : 0.0f)) * inv_seq;
    if (tcap) tcap[(size_t)t * V + v] = zv * ic;
  }
}

hipError_t ce_grad_views(const float* logits, const uint32_t* tgt, int T, int V, float inv_seq,
                         float softcap, float* dl, float* tcap, hipStream_t st) {
  if (T < 0 || V < 1) return hipErrorInvalidValue;
  if (T == 0 || (!dl && !tcap)) return hipSuccess;
  hipLaunchKernelGGL(ce_grad_views_kernel, dim3(T), dim3(256), 0, st, logits, tgt, V, inv_seq,
                     softcap > 0.f ? softcap : 0.f, dl, tcap);
  return hipGetLastError();
}

// x_prenorm and x_final = x * rinv * gamma (cpu/rmsnorm.rs:149-183 order) for
// token t = b*S + s, written channel-first per sequence: [b][c][s].
__global__ __launch_bounds__(256) void final_norm_views_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ rinv, int S,
                                                               int d, float* __restrict__ pre,
                                                               float* __restrict__ fin) {
  const int t = blockIdx.x, b = t / S, s = t - b * S;
  const float r = rinv[t];
  for (int c = threadIdx.x; c < d; c += 256) {
    const float v = x[(size_t)t * d + c];
    const size_t o = ((size_t)b * d + c) * S + s;
    if (pre) pre[o] = v;
    if (fin) fin[o] = v * r * gamma[c];
  }
}

hipError_t final_norm_views(const float* x, const float* gamma, const float* rinv, int B, int S, int d,
                            float* pre, float* fin, hipStream_t st) {
  if (B < 0 || S < 1 || d < 1) return hipErrorInvalidValue;
  if (B == 0 || (!pre && !fin)) return hipSuccess;
  hipLaunchKernelGGL(final_norm_views_kernel, dim3(B * S), dim3(256), 0, st, x, gamma, rinv, S, d, pre,
                     fin);
  return hipGetLastError();
}

// ---- RMSNorm backward -----------------------------------------------------------
// cpu/rmsnorm.rs:190-236 per row t, with r = 1/sqrt(mean(x^2) + eps)
// recomputed from x as the forward computes it:
//   x_hat = x r,  dot = sum_d dy gamma x_hat / dim,  dx = r (dy gamma - x_hat dot)
// out = res + dx (res nullable: the residual stream's own gradient), and
// rinv[t] = r for the gamma gradient below.
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const float* __restrict__ dy,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ gamma,
                                                          const float* res, float* out,
                                                          float* __restrict__ rinv, int dim,
                                                          float eps) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const float* xr = x + (size_t)t * dim;
  const float* dr = dy + (size_t)t * dim;
  float ss = 0.f;
  for (int i = threadIdx.x * 4; i < dim; i += 1024) {
    const f32x4 v = *(const f32x4*)(xr + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = block_sum<4>(ss, red);
  const float r = 1.0f / sqrtf(ss * (1.0f / (float)dim) + eps);
  float dot = 0.f;
  for (int i = threadIdx.x * 4; i < dim; i += 1024) {
    const f32x4 v = *(const f32x4*)(xr + i), d = *(const f32x4*)(dr + i),
                g = *(const f32x4*)(gamma + i);
    dot += d.x * g.x * (v.x * r) + d.y * g.y * (v.y * r) + d.z * g.z * (v.z * r) +
           d.w * g.w * (v.w * r);
  }
  dot = block_sum<4>(dot, red) * (1.0f / (float)dim);
  for (int i = threadIdx.x * 4; i < dim; i += 1024) {
    const f32x4 v = *(const f32x4*)(xr + i), d = *(const f32x4*)(dr + i),
                g = *(const f32x4*)(gamma + i);
    f32x4 o;
    o.x = r * (d.x * g.x - v.x * r * dot);
    o.y = r * (d.y * g.y - v.y * r * dot);
    o.z = r * (d.z * g.z - v.z * r * dot);
    o.w = r * (d.w * g.w - v.w * r * dot);
    if (res) {
      const f32x4 a = *(const f32x4*)(res + (size_t)t * dim + i);
      o.x += a.x;
      o.y += a.y;
      o.z += a.z;
      o.w += a.w;
    }
    *(f32x4*)(out + (size_t)t * dim + i) = o;
  }
  if (threadIdx.x == 0) rinv[t] = r;
}

// dgamma[d] += sum_t dy[t, d] x[t, d] rinv[t], in two fixed-order passes:
// NORM_PARTS partial sums over interleaved row sets, then their sum in order.
constexpr int NORM_PARTS = 64;
__global__ __launch_bounds__(256) void gamma_partial_kernel(const float* __restrict__ dy,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ rinv, int T,
                                                            int dim, float* __restrict__ part) {
  const int d = blockIdx.x * 256 + threadIdx.x, p = blockIdx.y;
  if (d >= dim) return;
  float s = 0.f;
  for (int t = p; t < T; t += NORM_PARTS) s += dy[(size_t)t * dim + d] * (x[(size_t)t * dim + d] * rinv[t]);
  part[(size_t)p * dim + d] = s;
}
__global__ __launch_bounds__(256) void gamma_reduce_kernel(const float* __restrict__ part, int dim,
                                                           float* __restrict__ dgamma, int acc,
                                                           float* __restrict__ sq) {
  __shared__ float red[4];
  const int d = blockIdx.x * 256 + threadIdx.x;
  float val = 0.f;
  if (d < dim) {
    float s = 0.f;
    for (int p = 0; p < NORM_PARTS; ++p) s += part[(size_t)p * dim + d];
    val = acc ? dgamma[d] + s : s;
    dgamma[d] = val;
  }
  if (sq) {
    const float t = block_sum<4>(val * val, red);
    if (threadIdx.x == 0) sq[blockIdx.x] = t;
  }
}

hipError_t rmsnorm_backward(const float* dy, const float* x, const float* gamma, const float* res,
                            int T, int dim, float eps, float* out, float* rinv, float* part,
                            float* dgamma, bool accumulate, hipStream_t st, float* sq) {
  if (T < 1 || dim < 4 || dim % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(rmsnorm_bwd_kernel, dim3(T), dim3(256), 0, st, dy, x, gamma, res, out, rinv, dim,
                     eps);
  hipLaunchKernelGGL(gamma_partial_kernel, dim3((dim + 255) / 256, NORM_PARTS), dim3(256), 0, st, dy,
                     x, rinv, T, dim, part);
  hipLaunchKernelGGL(gamma_reduce_kernel, dim3((dim + 255) / 256), dim3(256), 0, st, part, dim,
                     dgamma, accumulate ? 1 : 0, sq);
  return hipGetLastError();
}
size_t rmsnorm_backward_part_floats(int dim) { return (size_t)NORM_PARTS * dim; }

// ---- embedding backward -----------------------------------------------------------
// dE[tok[t]] += dx[t] (cpu/embedding.rs:34-44 scatter-add) without atomics:
// the workgroup of position t returns unless t is the first occurrence of its
// token; the first one sums the rows of every occurrence in position order
// and adds the sum to the row of dE, so the result does not depend on
// scheduling. Tokens are staged through LDS in chunks of EMB_CHUNK.
constexpr int EMB_CHUNK = 4096;
constexpr int EMB_MAX_DIM = 8192;  // 8 float4 per thread
__global__ __launch_bounds__(256) void embed_bwd_kernel(const float* __restrict__ dx,
                                                        const uint32_t* __restrict__ tok, int T,
                                                        int dim, int vocab,
                                                        float* __restrict__ dE) {
  __shared__ uint32_t st[EMB_CHUNK];
  const int t = blockIdx.x;
  const uint32_t v = tok[t];
  if (v >= (uint32_t)vocab) return;  // the forward's embedding kernel reports it
  int dup = 0;
  for (int u = threadIdx.x; u < t; u += 256) dup |= tok[u] == v;
  if (__syncthreads_or(dup)) return;
  f32x4 acc[EMB_MAX_DIM / 1024];
#pragma unroll
  for (int k = 0; k < EMB_MAX_DIM / 1024; ++k) acc[k] = f32x4{};
  for (int c0 = t; c0 < T; c0 += EMB_CHUNK) {
    const int n = min(EMB_CHUNK, T - c0);
    __syncthreads();
    for (int u = threadIdx.x; u < n; u += 256) st[u] = tok[c0 + u];
    __syncthreads();
    for (int u = 0; u < n; ++u) {
      if (st[u] != v) continue;
      const float* row = dx + (size_t)(c0 + u) * dim;
#pragma unroll
      for (int k = 0; k < EMB_MAX_DIM / 1024; ++k) {
        const int i = k * 1024 + threadIdx.x * 4;
        if (i < dim) {
          const f32x4 a = *(const f32x4*)(row + i);
          acc[k].x += a.x;
          acc[k].y += a.y;
          acc[k].z += a.z;
          acc[k].w += a.w;
        }
      }
    }
  }
  float* o = dE + (size_t)v * dim;
#pragma unroll
  for (int k = 0; k < EMB_MAX_DIM / 1024; ++k) {
    const int i = k * 1024 + threadIdx.x * 4;
    if (i < dim) {
      f32x4 e = *(f32x4*)(o + i);
      e.x += acc[k].x;
      e.y += acc[k].y;
      e.z += acc[k].z;
      e.w += acc[k].w;
      *(f32x4*)(o + i) = e;
    }
  }
}

hipError_t embedding_backward(const float* dx, const uint32_t* tok, int T, int dim, int vocab,
                              float* dE, hipStream_t st) {
  if (T < 0 || dim % 4 || dim > EMB_MAX_DIM) return hipErrorInvalidValue;
  if (T == 0) return hipSuccess;
  hipLaunchKernelGGL(embed_bwd_kernel, dim3(T), dim3(256), 0, st, dx, tok, T, dim, vocab, dE);
  return hipGetLastError();
}

}  // namespace hb
