// Optimizer kernels: fused AdamW over the fp32 master copy, the global
// gradient L2 norm and the clip scale.
//
// The optimizer's fp32 arenas (master weights, gradients, first and second
// moments) hold every tensor in the packed order of the fp16 weights the
// GEMMs read, element for element. One elementwise pass therefore updates
// param/m/v and rewrites the fp16 copy at the same index: 30 bytes per
// parameter (read param, grad, m, v; write param, m, v and the fp16 weight),
// HBM-bound. The reference's fused step (cpu/adam.rs:95-132, and the Metal
// shader of metal_adam.rs:13-38 with the same arithmetic) moves 28 bytes per
// parameter and keeps no second copy.
#include "internal.hpp"

namespace hb {

// cpu/adam.rs:119-131, one element:
//   g = grad * gscale; m = b1 m + (1-b1) g; v = b2 v + (1-b2) g g;
//   update = (m bc1) / (sqrt(v bc2) + eps); p -= lr (update + wd p)
// evaluated in that order with every operation rounded to fp32 (no fused
// multiply-adds), so results match the reference formula bit for bit where
// sqrt and division are correctly rounded, which they are here (no fast-math).
// Four consecutive elements; both kernels below evaluate exactly this.
HB_DEV void adamw4(const f32x4& pv, const f32x4& gv, const f32x4& mv, const f32x4& vv, float gs,
                   const AdamW& h, f32x4& po, f32x4& mo, f32x4& vo) {
#pragma clang fp contract(off)
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float gg = gv[e] * gs;
    const float a = h.b1 * mv[e];
    const float b = h.omb1 * gg;
    const float mi = a + b;
    const float c = h.b2 * vv[e];
    const float d = h.omb2 * gg;
    const float vi = c + d * gg;
    const float mh = mi * h.bc1;
    const float vh = vi * h.bc2;
    const float upd = mh / (sqrtf(vh) + h.eps);
    const float wdp = h.wd * pv[e];
    po[e] = pv[e] - h.lr * (upd + wdp);
    mo[e] = mi;
    vo[e] = vi;
  }
}

template <bool F16DST>
__global__ __launch_bounds__(256) void adamw_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                    float* __restrict__ m, float* __restrict__ v,
                                                    void* __restrict__ dst, size_t n4, AdamW h,
                                                    const float* __restrict__ d_gscale) {
  const float gs = d_gscale ? *d_gscale : h.gscale;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    // non-temporal loads: every operand is read once (7B step 34.5-35.0 ->
    // 34.0-34.1 ms); the stores stay ordinary (non-temporal stores measured
    // far slower for write streams)
    const f32x4 pv = __builtin_nontemporal_load(((const f32x4*)p) + i);
    const f32x4 gv = __builtin_nontemporal_load(((const f32x4*)g) + i);
    const f32x4 mv = __builtin_nontemporal_load(((const f32x4*)m) + i);
    const f32x4 vv = __builtin_nontemporal_load(((const f32x4*)v) + i);
    f32x4 po, mo, vo;
    adamw4(pv, gv, mv, vv, gs, h, po, mo, vo);
    ((f32x4*)p)[i] = po;
    ((f32x4*)m)[i] = mo;
    ((f32x4*)v)[i] = vo;
    if constexpr (F16DST) {
      f16x4 o;
      o.x = (f16)po.x;
      o.y = (f16)po.y;
      o.z = (f16)po.z;
      o.w = (f16)po.w;
      ((f16x4*)dst)[i] = o;
    } else {
      ((f32x4*)dst)[i] = po;
    }
  }
}

static int stream_blocks(size_t n4) {
  const size_t b = (n4 + 255) / 256;
  return (int)(b < 4096 ? b : 4096);
}

hipError_t adamw(float* p, const float* g, float* m, float* v, f16* dst16, float* dst32, size_t n,
                 const AdamW& h, const float* d_gscale, hipStream_t st) {
  if (n % 4 || (!dst16 && !dst32)) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  const size_t n4 = n / 4;
  if (dst16)
    hipLaunchKernelGGL(adamw_kernel<true>, dim3(stream_blocks(n4)), dim3(256), 0, st, p, g, m, v,
                       (void*)dst16, n4, h, d_gscale);
  else
    hipLaunchKernelGGL(adamw_kernel<false>, dim3(stream_blocks(n4)), dim3(256), 0, st, p, g, m, v,
                       (void*)dst32, n4, h, d_gscale);
  return hipGetLastError();
}

// One matrix [R][C] (packed order) in 64x64 tiles: the same update, the fp16
// weight written row-major (dst) and transposed (dstT [C][ldT], the copy the
// training backward's dX products read), so an optimizer step leaves both
// fp16 copies current without a separate transpose pass (+2 B per parameter
// instead of reading and writing 4). Rows [R, ldT) of dstT's tiles are zero.
__global__ __launch_bounds__(256) void adamw_tile_kernel(float* __restrict__ p,
                                                         const float* __restrict__ g,
                                                         float* __restrict__ m, float* __restrict__ v,
                                                         f16* __restrict__ dst, f16* __restrict__ dstT,
                                                         int R, int C, int ldT, AdamW h,
                                                         const float* __restrict__ d_gscale) {
  __shared__ f16x8 tile[64 * 9];  // [64 rows][72 halfs]
  const float gs = d_gscale ? *d_gscale : h.gscale;
  const int tid = threadIdx.x, c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
  const int tx = tid & 15, ty = tid >> 4;
  f16* t = (f16*)tile;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rl = ty + 16 * i, r = r0 + rl, c = c0 + tx * 4;
    f16x4 o = {};
    if (r < R && c < C) {
      const size_t idx = (size_t)r * C + c;
      const f32x4 pv = __builtin_nontemporal_load((const f32x4*)(p + idx));  // as adamw_kernel
      const f32x4 gv = __builtin_nontemporal_load((const f32x4*)(g + idx));
      const f32x4 mv = __builtin_nontemporal_load((const f32x4*)(m + idx));
      const f32x4 vv = __builtin_nontemporal_load((const f32x4*)(v + idx));
      f32x4 po, mo, vo;
      adamw4(pv, gv, mv, vv, gs, h, po, mo, vo);
      *(f32x4*)(p + idx) = po;
      *(f32x4*)(m + idx) = mo;
      *(f32x4*)(v + idx) = vo;
      o.x = (f16)po.x;
      o.y = (f16)po.y;
      o.z = (f16)po.z;
      o.w = (f16)po.w;
      *(f16x4*)(dst + idx) = o;
    }
    *(f16x4*)(t + rl * 72 + tx * 4) = o;
  }
  __syncthreads();
  const int lr = tid >> 3, lc = (tid & 7) * 8;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int cc = q * 32 + lr;
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = t[(lc + j) * 72 + cc];
    if (c0 + cc < C && r0 + lc < ldT) *(f16x8*)(dstT + (size_t)(c0 + cc) * ldT + r0 + lc) = o;
  }
}

hipError_t adamw_tiled(float* p, const float* g, float* m, float* v, f16* dst, f16* dstT, int R,
                       int C, int ldT, const AdamW& h, const float* d_gscale, hipStream_t st) {
  if (R < 1 || C < 4 || C % 4 || ldT < R || ldT % 8 || !dst || !dstT) return hipErrorInvalidValue;
  hipLaunchKernelGGL(adamw_tile_kernel, dim3((C + 63) / 64, (ldT + 63) / 64), dim3(256), 0, st, p, g,
                     m, v, dst, dstT, R, C, ldT, h, d_gscale);
  return hipGetLastError();
}

// ---- gradient norm from partial sums taken while the gradient was written ----
// Block i folds slots i, i + SUMSQ_BLOCKS, ... (each thread a fixed strided
// share, in fp64) and adds extra[i]: the same order on every run.
__global__ __launch_bounds__(256) void combine_sumsq_kernel(const float* __restrict__ slots, long n,
                                                            const double* __restrict__ extra,
                                                            double* __restrict__ partials) {
  __shared__ double red[4];
  double s = 0.0;
  for (long j = blockIdx.x + (long)SUMSQ_BLOCKS * threadIdx.x; j < n; j += (long)SUMSQ_BLOCKS * 256)
    s += (double)slots[j];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) partials[blockIdx.x] = red[0] + red[1] + red[2] + red[3] + extra[blockIdx.x];
}

hipError_t combine_sumsq(const float* slots, long n, const double* extra, double* partials,
                         hipStream_t st) {
  if (n < 0 || !extra || !partials) return hipErrorInvalidValue;
  hipLaunchKernelGGL(combine_sumsq_kernel, dim3(SUMSQ_BLOCKS), dim3(256), 0, st, slots, n, extra,
                     partials);
  return hipGetLastError();
}

// ---- global gradient norm (full_model.rs:600-622) ----------------------------
// A fixed grid of SUMSQ_BLOCKS workgroups, each summing a fixed strided share
// of the squares in fp64 and writing one partial: the same result on every
// run. (The reference sums per tensor in fp32 with vDSP_svesq; fp64 here
// keeps the norm of 6.6e9 terms accurate to the last fp32 bit or so.)
__global__ __launch_bounds__(256) void sumsq_kernel(const float* __restrict__ g, size_t n4,
                                                    double* __restrict__ partials) {
  __shared__ double red[4];
  double s = 0.0;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const f32x4 x = ((const f32x4*)g)[i];
    s += (double)x.x * x.x + (double)x.y * x.y + (double)x.z * x.z + (double)x.w * x.w;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) partials[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

hipError_t grad_sumsq(const float* g, size_t n, double* partials, hipStream_t st) {
  if (n % 4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(sumsq_kernel, dim3(SUMSQ_BLOCKS), dim3(256), 0, st, g, n / 4, partials);
  return hipGetLastError();
}

// out[0] = ||g|| (fp32), out[1] = the gradient scale train_step applies
// (full_model.rs:697-705): gsc when ||g|| * gsc <= clip, else clip / ||g||;
// out[2] = the clip_grads factor (full_model.rs:625-641): clip / ||g|| when
// ||g|| > clip, else 1.
__global__ __launch_bounds__(256) void clip_scale_kernel(const double* __restrict__ partials,
                                                         ClipCfg c, float* __restrict__ out) {
  __shared__ double red[256];
  double s = 0.0;
  for (int i = threadIdx.x; i < SUMSQ_BLOCKS; i += 256) s += partials[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
#pragma clang fp contract(off)
    const float raw = (float)sqrt(red[0]);
    const float scaled = raw * c.gsc;
    out[0] = raw;
    out[1] = scaled > c.grad_clip ? c.grad_clip / raw : c.gsc;
    out[2] = raw > c.grad_clip ? c.grad_clip / raw : 1.0f;
  }
}

hipError_t grad_clip_scale(const double* partials, ClipCfg c, float* out, hipStream_t st) {
  hipLaunchKernelGGL(clip_scale_kernel, dim3(1), dim3(256), 0, st, partials, c, out);
  return hipGetLastError();
}

// g *= *d_scale (clip_grads' sscal, full_model.rs:628-640).
__global__ __launch_bounds__(256) void scale_kernel(float* __restrict__ g, size_t n4,
                                                    const float* __restrict__ d_scale) {
  const float s = *d_scale;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    f32x4 x = ((f32x4*)g)[i];
    x.x *= s;
    x.y *= s;
    x.z *= s;
    x.w *= s;
    ((f32x4*)g)[i] = x;
  }
}

hipError_t scale_inplace(float* g, size_t n, const float* d_scale, hipStream_t st) {
  if (n % 4) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(scale_kernel, dim3(stream_blocks(n / 4)), dim3(256), 0, st, g, n / 4, d_scale);
  return hipGetLastError();
}

// dst[i] = (float)src[i]: the master copy of a model whose fp32 weights were
// never given to the optimizer starts from the fp16 values the GEMMs use.
__global__ __launch_bounds__(256) void widen_kernel(const f16* __restrict__ src, float* __restrict__ dst,
                                                    size_t n4) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const f16x4 h = ((const f16x4*)src)[i];
    ((f32x4*)dst)[i] = f32x4{(float)h.x, (float)h.y, (float)h.z, (float)h.w};
  }
}

hipError_t widen_f16(const f16* src, float* dst, size_t n, hipStream_t st) {
  if (n % 4) return hipErrorInvalidValue;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(widen_kernel, dim3(stream_blocks(n / 4)), dim3(256), 0, st, src, dst, n / 4);
  return hipGetLastError();
}

}  // namespace hb
