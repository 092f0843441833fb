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
// above the row-major kernel it replaced.
//
// A workgroup owns one 16-row block; its KS waves split K (deterministic LDS
// reduction at the end).
//
// Optional RMSNorm tail (decode residual projections): the epilogue writes the
// new fp32 residual rows with device-coherent (agent-scope) stores, and the
// last workgroup to finish (atomic ticket) normalises those rows into the fp16
// input of the next projection. This replaces a separate launch per norm.
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

// RMSNorm of the B rows [B, N] just written by the epilogue (cpu/rmsnorm.rs:
// 149-183: r = 1/sqrt(sum(x^2)/N + eps), y = x * r * gamma), run by the last
// workgroup. Rows are spread over the waves: G waves per row (G = KS/B rounded
// down to a power of two, at least 1), so B = 1 uses the whole workgroup and
// B >= KS one wave per row. Reads use agent-scope loads: the rows were written
// by other workgroups, possibly on other XCDs, with agent-scope stores.
//
// The tail sits on the critical path of the decode step, so it is built for
// latency: a lane issues all loads of a batch of up to CH 4-float chunks (and
// the matching gamma chunks) before using any, and when the row fits in one
// batch (N <= 1024*G: 8192 at B = 1) the output pass reuses those registers,
// leaving one memory round trip after the ticket. CH is small because the
// tail's registers count against the occupancy of the weight-streaming loop.
template <int KS>
HB_DEV void norm_tail(const NormTail& nt, int N, int B) {
  constexpr int CH = 4;
  __shared__ float s_red[KS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int G = KS;
  while (G > 1 && G * B > KS) G >>= 1;
  const int rows_per_pass = KS / G;
  const int part = wave % G;
  const int stride = G * 256;  // floats between a lane's consecutive chunks
  const int first = (part * 64 + lane) * 4;
  const bool one_batch = N <= stride * CH;
  auto ld = [](const float* a) {
    return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  f32x4 v[CH], g[CH];
  for (int row0 = 0; row0 < B; row0 += rows_per_pass) {
    const int row = row0 + wave / G;
    const bool ok = row < B;
    const float* xr = nt.x + (size_t)(ok ? row : 0) * N;
    float ss = 0.f;
    for (int c0 = first; c0 < N; c0 += stride * CH) {
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int c = c0 + i * stride;
        if (ok && c < N) {
          v[i].x = ld(xr + c);
          v[i].y = ld(xr + c + 1);
          v[i].z = ld(xr + c + 2);
          v[i].w = ld(xr + c + 3);
          g[i] = *(const f32x4*)(nt.gamma + c);
        } else {
          v[i] = f32x4{};
        }
      }
#pragma unroll
      for (int i = 0; i < CH; ++i)
        ss += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
    }
    ss = wave_sum(ss);
    __syncthreads();  // s_red reuse across passes
    if (lane == 0) s_red[wave] = ss;
    __syncthreads();
    if (ok) {
      float tot = 0.f;
      const int w0 = (wave / G) * G;
      for (int w = 0; w < G; ++w) tot += s_red[w0 + w];
      const float r = 1.0f / sqrtf(tot * (1.0f / (float)N) + nt.eps);
      f16* orow = nt.out + (size_t)row * N;
      for (int c0 = first; c0 < N; c0 += stride * CH) {
        if (!one_batch) {
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            const int c = c0 + i * stride;
            if (c < N) {
              v[i].x = ld(xr + c);
              v[i].y = ld(xr + c + 1);
              v[i].z = ld(xr + c + 2);
              v[i].w = ld(xr + c + 3);
              g[i] = *(const f32x4*)(nt.gamma + c);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < CH; ++i) {
          const int c = c0 + i * stride;
          if (c < N) {
            f16x4 o;
            o.x = (f16)(v[i].x * r * g[i].x);
            o.y = (f16)(v[i].y * r * g[i].y);
            o.z = (f16)(v[i].z * r * g[i].z);
            o.w = (f16)(v[i].w * r * g[i].w);
            *(f16x4*)(orow + c) = o;
          }
        }
      }
    }
  }
}

template <int KS, int U, class Epi, bool TAIL>
__global__ __launch_bounds__(KS * 64) void gemv_kernel(const f16x8* __restrict__ Wt,
                                                       const f16* __restrict__ X, int N, int B,
                                                       int K, Epi epi, NormTail nt) {
  __shared__ f32x4 red[KS][64];
  __shared__ int s_ticket;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rb = blockIdx.x;
  const int col = lane & 15, kq = 8 * (lane >> 4);
  const int nsteps = K >> 5;
  const int s_begin = (nsteps * wave) / KS, s_end = (nsteps * (wave + 1)) / KS;
  const f16x8* wp = Wt + (size_t)rb * nsteps * 64 + lane;
  const bool xok = col < B;
  const f16* xrow = X + (size_t)(xok ? col : 0) * K + kq;

  f32x4 acc = {};
  const f16x8 zero8 = {};
  int s = s_begin;
  for (; s + U <= s_end; s += U) {
    f16x8 a[U], bx[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      a[u] = __builtin_nontemporal_load(wp + (size_t)(s + u) * 64);
      bx[u] = xok ? *(const f16x8*)(xrow + (size_t)(s + u) * 32) : zero8;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], bx[u], acc, 0, 0, 0);
  }
  for (; s < s_end; ++s) {
    const f16x8 a = __builtin_nontemporal_load(wp + (size_t)s * 64);
    const f16x8 bx = xok ? *(const f16x8*)(xrow + (size_t)s * 32) : zero8;
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bx, acc, 0, 0, 0);
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
  }
  if constexpr (TAIL) {
    // Every store of this workgroup has completed before the ticket is taken.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0)
      s_ticket = (int)__builtin_amdgcn_atomic_inc32(nt.counter, gridDim.x - 1, __ATOMIC_RELAXED,
                                                    "agent");
    __syncthreads();
    if (s_ticket != (int)gridDim.x - 1) return;
    norm_tail<KS>(nt, N, B);
  }
}

namespace {
constexpr int GEMV_KS = 8;  // waves per workgroup (K split)
constexpr int GEMV_U = 4;   // 1 KB weight loads in flight per wave

template <class Epi, bool TAIL = false>
hipError_t launch_gemv(const f16* Wt, const f16* X, int N, int B, int K, const Epi& epi,
                       const NormTail& nt, hipStream_t st) {
  if (B < 1 || B > 16 || N % 16 || K % 32) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemv_kernel<GEMV_KS, GEMV_U, Epi, TAIL>), dim3(N / 16), dim3(GEMV_KS * 64), 0,
                     st, (const f16x8*)Wt, X, N, B, K, epi, nt);
  return hipGetLastError();
}
}  // namespace

hipError_t gemv_residual(const f16* Wt, const f16* X, int N, int B, int K, const EpiResidual& e,
                         hipStream_t st) {
  return launch_gemv(Wt, X, N, B, K, e, NormTail{}, st);
}
hipError_t gemv_residual_norm(const f16* Wt, const f16* X, int N, int B, int K,
                              const EpiResidual& e, const NormTail& nt, hipStream_t st) {
  if (nt.x != e.out || !nt.gamma || !nt.out || !nt.counter) return hipErrorInvalidValue;
  return launch_gemv<EpiResidualCoherent, true>(Wt, X, N, B, K, EpiResidualCoherent{e}, nt, st);
}
hipError_t gemv_swiglu(const f16* Wt, const f16* X, int N, int B, int K, const EpiSwiGLU& e,
                       hipStream_t st) {
  return launch_gemv(Wt, X, N, B, K, e, NormTail{}, st);
}
hipError_t gemv_logits(const f16* Wt, const f16* X, int N, int B, int K, const EpiLogits& e,
                       hipStream_t st) {
  return launch_gemv(Wt, X, N, B, K, e, NormTail{}, st);
}
hipError_t gemv_qkv(const f16* Wt, const f16* X, int N, int B, int K, const EpiQKV& e,
                    hipStream_t st) {
  return launch_gemv(Wt, X, N, B, K, e, NormTail{}, st);
}
hipError_t gemv_store(const f16* Wt, const f16* X, int N, int B, int K, float* C, hipStream_t st) {
  return launch_gemv(Wt, X, N, B, K, EpiStore{C, N}, NormTail{}, st);
}

}  // namespace hb
