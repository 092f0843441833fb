// Bandwidth-bound kernels: embedding gather, RMSNorm, cross-entropy/argmax,
// reductions, weight repacking and the seeded synthetic fill.
#include "internal.hpp"
#include "synth.hpp"

namespace hb {

// ---- embedding (cpu/embedding.rs:8-16): x[t,:] = E[tok[t],:] -------------------
__global__ __launch_bounds__(256) void embedding_kernel(const f16* __restrict__ E,
                                                        const uint32_t* __restrict__ tok, int dim,
                                                        int vocab, float* __restrict__ x,
                                                        int* err) {
  const int t = blockIdx.x;
  const uint32_t id = tok[t];
  float* xr = x + (size_t)t * dim;
  if (id >= (uint32_t)vocab) {
    // Never read outside E; report through the error word.
    for (int c = threadIdx.x * 4; c < dim; c += 256 * 4) *(f32x4*)(xr + c) = f32x4{};
    if (threadIdx.x == 0 && err) atomicOr(err, 1);
    return;
  }
  const f16* er = E + (size_t)id * dim;
  for (int c = threadIdx.x * 8; c < dim; c += 256 * 8) {
    const f16x8 v = *(const f16x8*)(er + c);
    f32x4 a, b;
    a.x = (float)v[0]; a.y = (float)v[1]; a.z = (float)v[2]; a.w = (float)v[3];
    b.x = (float)v[4]; b.y = (float)v[5]; b.z = (float)v[6]; b.w = (float)v[7];
    *(f32x4*)(xr + c) = a;
    *(f32x4*)(xr + c + 4) = b;
  }
}

hipError_t embedding(const f16* E, const uint32_t* tok, int T, int dim, int vocab, float* x,
                     int* err, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(embedding_kernel, dim3(T), dim3(256), 0, st, E, tok, dim, vocab, x, err);
  return hipGetLastError();
}

// ---- RMSNorm (cpu/rmsnorm.rs:149-183) -------------------------------------------
// r = 1/sqrt(sum(x^2) * (1/dim) + eps); y = x * r * gamma. One workgroup per row.
// NPT > 0: dim = NPT * 1024, each thread owns NPT float4 chunks, all loads are
// issued before any use and the row stays in registers for the second pass.
// NPT = 0: any dim (multiple of 4), strided loop. Both add each thread's
// squares in the same order, so the result does not depend on the variant.
// NPT > 0: dim = NPT * 1024 held in registers; RAG: dim <= NPT * 1024 (dim % 4
// == 0), the chunks past dim skipped (they add 0 to the sum of squares, which
// leaves it unchanged, so the result equals the two-pass NPT = 0 form's).
template <int NPT, bool RAG = false>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x, long row_stride,
                                                      const float* __restrict__ gamma, int dim,
                                                      float eps, f16* __restrict__ out,
                                                      float* __restrict__ rms_inv, int split) {
  __shared__ float red[4];
  const int t = blockIdx.x;
  const float* xr = x + (size_t)t * row_stride;
  f16* orow = out + (size_t)t * dim * (split ? 2 : 1);
  const size_t lo = split ? (size_t)dim : 0;  // split rows: [hi | lo]
  float ss = 0.f;
  if constexpr (NPT > 0) {
    auto in = [&](int i) { return !RAG || (int)threadIdx.x * 4 + i * 1024 < dim; };
    f32x4 v[NPT], g[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) v[i] = in(i) ? *(const f32x4*)(xr + threadIdx.x * 4 + i * 1024) : f32x4{};
#pragma unroll
    for (int i = 0; i < NPT; ++i) g[i] = in(i) ? *(const f32x4*)(gamma + threadIdx.x * 4 + i * 1024) : f32x4{};
#pragma unroll
    for (int i = 0; i < NPT; ++i) ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    ss = block_sum<4>(ss, red);
    const float r = 1.0f / sqrtf(ss * (1.0f / (float)dim) + eps);
    if (rms_inv && threadIdx.x == 0) rms_inv[t] = r;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      if (!in(i)) continue;
      f32x4 o;
      o.x = v[i].x * r * g[i].x;
      o.y = v[i].y * r * g[i].y;
      o.z = v[i].z * r * g[i].z;
      o.w = v[i].w * r * g[i].w;
      const int c = threadIdx.x * 4 + i * 1024;
      if (split == 2)  // the decode GEMVs' B-fragment order (EpiSwiGLU::frag), t < 16
        *(f16x4*)(out + ((size_t)(c >> 5) * 64 + t + 16 * ((c & 31) >> 3)) * 8 + (c & 7)) = f16x4_hi(o);
      else
        store_f16x4(orow + c, o, lo);
    }
  } else {
    for (int c = threadIdx.x * 4; c < dim; c += 1024) {
      const f32x4 v = *(const f32x4*)(xr + c);
      ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = block_sum<4>(ss, red);
    const float r = 1.0f / sqrtf(ss * (1.0f / (float)dim) + eps);
    if (rms_inv && threadIdx.x == 0) rms_inv[t] = r;
    for (int c = threadIdx.x * 4; c < dim; c += 1024) {
      const f32x4 v = *(const f32x4*)(xr + c);
      const f32x4 g = *(const f32x4*)(gamma + c);
      f32x4 o;
      o.x = v.x * r * g.x;
      o.y = v.y * r * g.y;
      o.z = v.z * r * g.z;
      o.w = v.w * r * g.w;
      if (split == 2)
        *(f16x4*)(out + ((size_t)(c >> 5) * 64 + t + 16 * ((c & 31) >> 3)) * 8 + (c & 7)) = f16x4_hi(o);
      else
        store_f16x4(orow + c, o, lo);
    }
  }
}

hipError_t rmsnorm(const float* x, long row_stride, const float* gamma, int T, int dim, float eps,
                   f16* out, float* rms_inv, hipStream_t st, bool split, bool frag) {
  if (T <= 0) return hipSuccess;
  if (frag && (split || T > 16 || dim % 32)) return hipErrorInvalidValue;
  const int sp = frag ? 2 : split ? 1 : 0;
  // 1..8: whole multiples of 1024; 9..16: ragged, ceil(dim / 1024) = 1..8
  const int np = dim % 1024 == 0 ? dim / 1024 : dim % 4 == 0 && dim < 8192 ? 8 + dim / 1024 + 1 : 0;
  switch (np) {
#define HB_NORM(n, c, rag)                                                                      \
  case c:                                                                                       \
    hipLaunchKernelGGL((rmsnorm_kernel<n, rag>), dim3(T), dim3(256), 0, st, x, row_stride, gamma, \
                       dim, eps, out, rms_inv, sp);                                             \
    break;
    HB_NORM(1, 1, false) HB_NORM(2, 2, false) HB_NORM(3, 3, false) HB_NORM(4, 4, false)
    HB_NORM(5, 5, false) HB_NORM(6, 6, false) HB_NORM(7, 7, false) HB_NORM(8, 8, false)
    HB_NORM(1, 9, true) HB_NORM(2, 10, true) HB_NORM(3, 11, true) HB_NORM(4, 12, true)
    HB_NORM(5, 13, true) HB_NORM(6, 14, true) HB_NORM(7, 15, true) HB_NORM(8, 16, true)
#undef HB_NORM
    default:
      hipLaunchKernelGGL(rmsnorm_kernel<0>, dim3(T), dim3(256), 0, st, x, row_stride, gamma, dim,
                         eps, out, rms_inv, sp);
  }
  return hipGetLastError();
}

// ---- cross-entropy (cpu/cross_entropy.rs:13-38, 58-96) ---------------------------
// One workgroup per row, one pass over the logits. Each thread takes its
// elements (4 consecutive per 1024) in batches of 8 float4 whose loads are
// issued together, raises its running maximum m once per batch (rescaling its
// sum of exp(x - m) then) and adds the batch's terms. The (m, sum) pairs are
// merged across the wave (LDS permutes) and across the 4 waves in LDS;
// loss = ln(sum) - (x[y] - max). The earlier form, one dependent load and
// branchy update per float4, took 29 us for 512 rows of 32000.
struct SoftState {
  float m, s;
};
HB_DEV void soft_merge(SoftState& a, const SoftState& b) {
  const float m = fmaxf(a.m, b.m);
  float s = 0.f;
  if (a.m != -INFINITY) s += a.s * exp2f((a.m - m) * HB_LOG2E);
  if (b.m != -INFINITY) s += b.s * exp2f((b.m - m) * HB_LOG2E);
  a.m = m;
  a.s = s;
}

__global__ __launch_bounds__(256) void cross_entropy_kernel(const float* __restrict__ logits,
                                                            const uint32_t* __restrict__ targets,
                                                            int vocab, float* __restrict__ loss,
                                                            int* err) {
  constexpr int NB = 8;  // float4 per thread and batch
  __shared__ SoftState red[4];
  const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float* row = logits + (size_t)t * vocab;
  SoftState st{-INFINITY, 0.f};
  for (int c0 = threadIdx.x * 4; c0 < vocab; c0 += NB * 1024) {
    f32x4 v[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int c = c0 + i * 1024;
      v[i] = c < vocab ? *(const f32x4*)(row + c) : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
    float bm = -INFINITY;  // c0 < vocab: v[0] holds real logits
#pragma unroll
    for (int i = 0; i < NB; ++i) bm = fmaxf(bm, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
    if (bm > st.m) {
      st.s *= exp2f((st.m - bm) * HB_LOG2E);  // 0 while st.m is -inf
      st.m = bm;
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < NB; ++i)
      acc += (exp2f((v[i].x - st.m) * HB_LOG2E) + exp2f((v[i].y - st.m) * HB_LOG2E)) +
             (exp2f((v[i].z - st.m) * HB_LOG2E) + exp2f((v[i].w - st.m) * HB_LOG2E));
    st.s += acc;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    SoftState b;
    b.m = __shfl_xor(st.m, o, 64);
    b.s = __shfl_xor(st.s, o, 64);
    soft_merge(st, b);
  }
  if (lane == 0) red[wave] = st;
  __syncthreads();
  if (threadIdx.x == 0) {
    SoftState r = red[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) soft_merge(r, red[w]);
    if (loss && targets) {
      const uint32_t y = targets[t];
      if (y < (uint32_t)vocab) {
        loss[t] = logf(r.s) - (row[y] - r.m);
      } else {
        loss[t] = NAN;
        if (err) atomicOr(err, 2);
      }
    }
  }
}

hipError_t cross_entropy(const float* logits, const uint32_t* targets, int T, int vocab,
                         float* loss, int* err, hipStream_t st) {
  if (T <= 0) return hipSuccess;
  hipLaunchKernelGGL(cross_entropy_kernel, dim3(T), dim3(256), 0, st, logits, targets, vocab, loss,
                     err);
  return hipGetLastError();
}

// Deterministic mean: fixed-order per-thread sums, fixed tree.
__global__ __launch_bounds__(256) void mean_kernel(const float* __restrict__ v, int n,
                                                   float* __restrict__ out) {
  __shared__ float red[4];
  float s = 0.f;
  for (int i = threadIdx.x; i < n; i += 256) s += v[i];
  s = block_sum<4>(s, red);
  if (threadIdx.x == 0) out[0] = s / (float)n;
}

hipError_t mean_reduce(const float* v, int n, float* out, hipStream_t st) {
  hipLaunchKernelGGL(mean_kernel, dim3(1), dim3(256), 0, st, v, n, out);
  return hipGetLastError();
}

__global__ void set_int_kernel(int* d, int v) { *d = v; }
hipError_t set_int(int* d, int value, hipStream_t st) {
  hipLaunchKernelGGL(set_int_kernel, dim3(1), dim3(1), 0, st, d, value);
  return hipGetLastError();
}

// ---- weight repacking -------------------------------------------------------------
HB_DEV int repack_row(int mode, int i, int j, int row0) {
  if (mode == 0) return row0 + j;
  if (mode == 1) return ((j >> 1) << 2) + (j & 1) + row0;
  return row0 + i;
}

// 64x64 tiles through LDS so both the fp32 reads and the writes are coalesced.
// D is f16 (the weights the GEMMs read) or float (the optimizer's fp32 master
// copy, stored in the same packed order).
template <class D>
__global__ __launch_bounds__(256) void repack_kernel(const float* __restrict__ src, int R, int C,
                                                     D* __restrict__ dst, int ld, int row0,
                                                     int mode) {
  __shared__ float tile[64][65];
  const int i0 = blockIdx.y * 64, j0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int i = i0 + r, j = j0 + tx;
    tile[r][tx] = (i < R && j < C) ? src[(size_t)i * C + j] : 0.f;
  }
  __syncthreads();
  if (mode == 2) {
    for (int r = ty; r < 64; r += 4) {
      const int i = i0 + r, j = j0 + tx;
      if (i < R && j < C) dst[(size_t)repack_row(mode, i, j, row0) * ld + j] = (D)tile[r][tx];
    }
  } else {
    // dst row indexed by source column j, dst column = source row i.
    for (int r = ty; r < 64; r += 4) {
      const int j = j0 + r, i = i0 + tx;
      if (i < R && j < C) dst[(size_t)repack_row(mode, i, j, row0) * ld + i] = (D)tile[tx][r];
    }
  }
}

hipError_t repack(const float* src, int R, int C, f16* dst, int ld, int row0, int mode,
                  hipStream_t st) {
  dim3 grid((C + 63) / 64, (R + 63) / 64);
  hipLaunchKernelGGL(repack_kernel<f16>, grid, dim3(256), 0, st, src, R, C, dst, ld, row0, mode);
  return hipGetLastError();
}

hipError_t repack_f32(const float* src, int R, int C, float* dst, int ld, int row0, int mode,
                      hipStream_t st) {
  dim3 grid((C + 63) / 64, (R + 63) / 64);
  hipLaunchKernelGGL(repack_kernel<float>, grid, dim3(256), 0, st, src, R, C, dst, ld, row0, mode);
  return hipGetLastError();
}

// Synthetic values of hb_synth_normal's sequence, elements [first, first+n),
// written as fp32 (the fp16 conversion then happens in repack_kernel, exactly
// as for a host upload of the same array).
__global__ __launch_bounds__(256) void synth_f32_kernel(uint64_t key, float scale, uint64_t first,
                                                        size_t n, float* __restrict__ dst) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    dst[i] = hb_normal_value(key, first + i, scale);
}

hipError_t synth_f32(uint64_t seed, uint64_t tensor_id, float scale, uint64_t first, size_t n,
                     float* dst, hipStream_t st) {
  const uint64_t key = hb_stream_key(seed, tensor_id);
  const int blocks = (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(synth_f32_kernel, dim3(blocks), dim3(256), 0, st, key, scale, first, n, dst);
  return hipGetLastError();
}

__global__ void fill_f32_kernel(float* d, float v, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    d[i] = v;
}
hipError_t fill_f32(float* d, float v, size_t n, hipStream_t st) {
  const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_f32_kernel, dim3(blocks), dim3(256), 0, st, d, v, n);
  return hipGetLastError();
}
__global__ void fill_f16_zero_kernel(f16* d, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    d[i] = (f16)0.f;
}
hipError_t fill_f16_zero(f16* d, size_t n, hipStream_t st) {
  const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_f16_zero_kernel, dim3(blocks), dim3(256), 0, st, d, n);
  return hipGetLastError();
}

// ---- validation windows (bin/train.rs:123-163, data.rs) --------------------------
// Window w = vs0 + b starts at pos = (w * S) % max_pos of the uint16 token
// stream (train.rs:135-137): inputs tokens[pos, pos+S), targets shifted by
// one. pos + S < max_pos + S = n - 1, so every read is inside the stream.
__global__ __launch_bounds__(256) void window_gather_kernel(const uint16_t* __restrict__ toks,
                                                            uint32_t vs0, int S, uint64_t max_pos,
                                                            uint32_t* __restrict__ tok,
                                                            uint32_t* __restrict__ tgt) {
  const int b = blockIdx.x;
  const uint64_t pos = ((uint64_t)(vs0 + (uint32_t)b) * (uint64_t)S) % max_pos;
  for (int s = threadIdx.x; s < S; s += 256) {
    tok[(size_t)b * S + s] = toks[pos + s];
    tgt[(size_t)b * S + s] = toks[pos + 1 + s];
  }
}

hipError_t window_gather(const uint16_t* toks, uint64_t n, uint32_t vs0, int B, int S,
                         uint32_t* tok, uint32_t* tgt, hipStream_t st) {
  if (B < 1 || S < 1 || n < (uint64_t)S + 2) return hipErrorInvalidValue;
  hipLaunchKernelGGL(window_gather_kernel, dim3(B), dim3(256), 0, st, toks, vs0, S,
                     n - (uint64_t)S - 1, tok, tgt);
  return hipGetLastError();
}

// acc[0] += sum of loss[0, T); with a byte-length table (data.rs:61-83):
// acc[1] += sum of loss[i] over targets with tb[target] > 0 and acc[2] += the
// sum of those byte lengths. One workgroup, fixed summation order (fp64), so
// the totals do not depend on scheduling.
__global__ __launch_bounds__(256) void bpb_accum_kernel(const float* __restrict__ loss,
                                                        const uint32_t* __restrict__ tgt, int T,
                                                        const int* __restrict__ tb, int tb_len,
                                                        double* __restrict__ acc) {
  __shared__ double red[3][256];
  double l = 0.0, nats = 0.0, bytes = 0.0;
  for (int i = threadIdx.x; i < T; i += 256) {
    const float x = loss[i];
    l += x;
    if (tb) {
      const uint32_t t = tgt[i];
      const int bl = t < (uint32_t)tb_len ? tb[t] : 0;
      if (bl > 0) {
        nats += x;
        bytes += bl;
      }
    }
  }
  red[0][threadIdx.x] = l;
  red[1][threadIdx.x] = nats;
  red[2][threadIdx.x] = bytes;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w)
      for (int k = 0; k < 3; ++k) red[k][threadIdx.x] += red[k][threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0)
    for (int k = 0; k < 3; ++k) acc[k] += red[k][0];
}

hipError_t bpb_accum(const float* loss, const uint32_t* tgt, int T, const int* tb, int tb_len,
                     double* acc, hipStream_t st) {
  if (T < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(bpb_accum_kernel, dim3(1), dim3(256), 0, st, loss, tgt, T, tb, tb_len, acc);
  return hipGetLastError();
}

}  // namespace hb
