// Shared types and device helpers for the gfx950 kernels of libhip_bridge.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define HB_DEV __device__ __forceinline__

// 1/ln(2): softmax is evaluated as exp2((s - m) * log2(e)).
#define HB_LOG2E 1.4426950408889634f

// n / d for 0 <= n < 2^31 and a divisor d >= 1 fixed at launch, by
// multiply-high (division by invariant integers, Granlund & Montgomery 1994):
//   s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1, q = (mulhi(n, m) + n) >> s.
// n + mulhi(n, m) < 2^32 because m < 2^32 and n < 2^31.
struct FastDiv {
  uint32_t d = 1, m = 1, s = 0;
  FastDiv() = default;
  __host__ explicit FastDiv(uint32_t dd) : d(dd) {
    while ((1ull << s) < dd) ++s;
    m = (uint32_t)(((1ull << 32) * ((1ull << s) - dd)) / dd + 1);
  }
  HB_DEV int div(int n) const { return (int)((__umulhi((uint32_t)n, m) + (uint32_t)n) >> s); }
};

// Decode-attention chunks at position pos (keys 0..pos) for n chunks per
// (sequence, head): chunk c holds keys [c * len, min((c + 1) * len, pos + 1))
// with len = ceil((pos + 1) / n); the first ceil((pos + 1) / len) <= n chunks
// hold keys. The attention kernel, the Wo GEMV's combine prologue and the
// combine kernel all take the split from here.
__host__ __device__ inline int attn_chunk_keys(int pos, int n) { return (pos + n) / n; }
__host__ __device__ inline int attn_chunks_valid(int pos, int n) {
  const int len = attn_chunk_keys(pos, n);
  return (pos + len) / len;
}

// x with bits 2 and 3 swapped: the key (or query) held in row slot x of a
// 32x32 MFMA tile whose A rows were loaded in that order, so that the 8
// accumulator registers 8j..8j+7 of lane half h hold the consecutive
// entries 16j+8h .. 16j+8h+7 (attention kernels).
HB_DEV int swap23(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

// LDS-only workgroup barrier: orders LDS accesses of the workgroup without
// draining outstanding global loads (a full __syncthreads would wait for the
// prefetches that are meant to stay in flight across it).
HB_DEV void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wave-wide reductions (64 lanes). __shfl_xor lowers to an LDS permute
// (ds_bpermute) and its wait; the register forms below avoid that in inner
// loops.
HB_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
HB_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Cross-lane steps in registers, without an LDS permute and its wait.
// dpp_f: a DPP lane permutation within each 16-lane row. group_sum<N>: the
// sum over each aligned group of N = 8 or 16 lanes, equal in every lane of
// the group (lane ^ 1, lane ^ 2, then the mirror image in the 8 and the 16,
// which meet the other quad / half once each quad / half is uniform).
// xor16_op / xor32_op: op(v[l], v[l ^ 16]) (or ^ 32) in every lane.
// v_permlane{16,32}_swap exchanges 16- or 32-lane halves of the wave between
// two registers; swapping two copies of v leaves one half of each pair
// broadcast in each register, and op commutes, so lane and partner agree.
template <int CTRL>
HB_DEV float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int N>
HB_DEV float group_sum(float v) {
  static_assert(N == 8 || N == 16, "groups of 8 or 16 lanes");
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  if constexpr (N == 16) v += dpp_f<0x140>(v);  // row_mirror
  return v;
}
template <class Op>
HB_DEV float xor16_op(float v, Op op) {
  const auto h = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(h[0]), __uint_as_float(h[1]));
}
template <class Op>
HB_DEV float xor32_op(float v, Op op) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(h[0]), __uint_as_float(h[1]));
}
// op over the lanes l, l ^ G, l ^ 2G, ... (G = 8 or 16): combines the
// groups of G lanes position by position, in every lane.
template <int G, class Op>
HB_DEV float fold_groups(float v, Op op) {
  static_assert(G == 8 || G == 16, "groups of 8 or 16 lanes");
  if constexpr (G == 8) v = op(v, dpp_f<0x128>(v));  // row_ror:8, lane ^ 8 within the row
  v = xor16_op(v, op);
  return xor32_op(v, op);
}

// Block-wide reduction through LDS; `red` holds one float per wave.
template <int NWAVES>
HB_DEV float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < NWAVES; ++w) s += red[w];
  return s;
}
template <int NWAVES>
HB_DEV float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < NWAVES; ++w) m = fmaxf(m, red[w]);
  return m;
}

// Workgroups are dispatched round-robin over the 8 XCDs (wg % 8). Remap so
// that each XCD receives a contiguous range of tile ids: tiles that share a
// weight panel then run on one XCD and share its L2. Bijective for any n.
HB_DEV int xcd_remap(int wg, int n) {
  const int q = n >> 3, r = n & 7;
  const int xcd = wg & 7, slot = wg >> 3;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
}

// silu(x) = x * sigmoid(x). The sigmoid keeps the IEEE division: through
// v_rcp_f32 (1 ulp) it made the 7B B=8 FFN-up GEMM 1% faster but moved the
// pooled top-1 agreement with the oracle from 99.62% to 99.57%.
HB_DEV float silu_f(float x) { return x * (1.0f / (1.0f + __expf(-x))); }

// Two-term fp16 form of fp32 values, for the operands that must carry more
// than fp16's 11 significant bits into an MFMA: x ~ hi + lo with hi = fp16(x)
// and lo = fp16(x - hi) (x - hi is exact in fp32), about 22 bits in all. An
// activation row of K features is then stored as 2K halves, [hi | lo], and a
// product with it runs the k-steps of hi and of lo against the same weights
// into the same fp32 accumulator ("split" rows).
HB_DEV f16x4 f16x4_hi(f32x4 v) {
  f16x4 h;
  h.x = (f16)v.x;
  h.y = (f16)v.y;
  h.z = (f16)v.z;
  h.w = (f16)v.w;
  return h;
}
HB_DEV f16x4 f16x4_lo(f32x4 v, f16x4 h) {
  f16x4 l;
  l.x = (f16)(v.x - (float)h.x);
  l.y = (f16)(v.y - (float)h.y);
  l.z = (f16)(v.z - (float)h.z);
  l.w = (f16)(v.w - (float)h.w);
  return l;
}
// Stores fp16(v) at p and, for split rows, its low part lo_off halves later.
HB_DEV void store_f16x4(f16* p, f32x4 v, size_t lo_off) {
  const f16x4 h = f16x4_hi(v);
  *(f16x4*)p = h;
  if (lo_off) *(f16x4*)(p + lo_off) = f16x4_lo(v, h);
}
