// GEMM epilogues. Both the prefill MFMA GEMM and the decode GEMV hand each
// lane's results to an epilogue as (token row t, first feature f0, 4 values
// for features f0..f0+3). f0 is always a multiple of 4, and feature blocks of
// 4 never straddle a Q/K/V or head boundary because hd % 64 == 0.
#pragma once
#include "common.hpp"

namespace hb {

// C[t, f0..f0+3] = v (fp32). Plain GEMM output.
struct EpiStore {
  float* c;
  int ldc;
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    *(f32x4*)(c + (size_t)t * ldc + f0) = v;
  }
};

// Split-K partial sums of the prefill GEMM: split blockIdx.y writes
// p[blockIdx.y * split_stride + t * ld + f0 ..]; splitk_reduce (gemm.hip) adds
// the splits in order and applies the real epilogue.
struct EpiSplit {
  float* p;
  int ld;
  size_t split_stride;
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    *(f32x4*)(p + blockIdx.y * split_stride + (size_t)t * ld + f0) = v;
  }
};

// out = res + alpha * v (fp32 residual stream). woFwd + vsma (layer.rs:784) and
// the ffnFused residual (kernels/ffn_fused.rs:74-77). The prefill GEMM loads
// the residual quads (load) for a group of quads before storing any of them;
// res may be the same buffer as out.
struct EpiResidual {
  const float* res;
  float* out;
  int ld;
  float alpha;
  using Aux = f32x4;
  HB_DEV f32x4 load(int t, int f0, int = 0) const { return *(const f32x4*)(res + (size_t)t * ld + f0); }
  HB_DEV void operator()(int t, int f0, f32x4 v, const f32x4& r, int = 0) const {
    f32x4 y;
    y.x = v.x * alpha + r.x;
    y.y = v.y * alpha + r.y;
    y.z = v.z * alpha + r.z;
    y.w = v.w * alpha + r.w;
    *(f32x4*)(out + (size_t)t * ld + f0) = y;
  }
  HB_DEV void operator()(int t, int f0, f32x4 v) const { (*this)(t, f0, v, load(t, f0)); }
};

// W1 and W3 are packed row-interleaved in groups of four: packed rows 4j..4j+3
// are W1 column 2j, W1 column 2j+1, W3 column 2j, W3 column 2j+1. A lane's
// 4 consecutive features are therefore (h1[u], h1[u+1], h3[u], h3[u+1]) with
// u = f0/2, and the SwiGLU gate (kernels/ffn_fused.rs:60-62) is formed in
// registers: gate = silu(h1) * h3.
struct EpiSwiGLU {
  f16* gate;   // [T, hidden]
  float* tap;  // nullable [T, 2*hidden] = h1 | h3
  int hidden;
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    const int u = f0 >> 1;
    f16x2 g;
    g.x = (f16)(silu_f(v.x) * v.z);
    g.y = (f16)(silu_f(v.y) * v.w);
    *(f16x2*)(gate + (size_t)t * hidden + u) = g;
    if (tap) {
      float* r = tap + (size_t)t * 2 * hidden;
      r[u] = v.x;
      r[u + 1] = v.y;
      r[hidden + u] = v.z;
      r[hidden + u + 1] = v.w;
    }
  }
};

// Tied-embedding logits with optional softcap (full_model.rs:228-239).
// The decode GEMV can also emit per-row-block argmax partials of the stored
// values (part_val/part_idx [B][N/16], nullable; see gemv.hip).
struct EpiLogits {
  float* logits;
  int vocab;
  float softcap;  // 0 = off
  float* part_val = nullptr;
  int* part_idx = nullptr;
  HB_DEV f32x4 capped(f32x4 v) const {
    if (softcap > 0.f) {
      const float ic = 1.0f / softcap;
      v.x = softcap * tanhf(v.x * ic);
      v.y = softcap * tanhf(v.y * ic);
      v.z = softcap * tanhf(v.z * ic);
      v.w = softcap * tanhf(v.w * ic);
    }
    return v;
  }
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    *(f32x4*)(logits + (size_t)t * vocab + f0) = capped(v);
  }
};

// Fused-QKV epilogue (kernels/sdpa_fwd.rs:70-128): the packed weight has Wq,
// Wk, Wv output rows stacked, so features [0,q) are Q, [q,q+kv) K, the rest V.
// Q and K get the interleaved RoPE of sdpa_fwd.rs:18-33 / 105-128 on pairs
// (2i, 2i+1) — both elements of a pair are in the same lane:
//   out[2i] = x[2i] c - x[2i+1] s,   out[2i+1] = x[2i+1] c + x[2i] s.
// Token t is position s = pos0 + t % S of sequence b = t / S (prefill), or
// position *d_pos of sequence b = t (decode, S = 1, pos0 read from d_pos).
struct EpiQKV {
  int q_dim, kv_dim, hd, S, heads, kv_heads;
  const float2* rope;  // [hd/2][rope_ld] (cos, sin), pair-major
  int rope_ld;         // positions per pair row
  const int* d_pos;    // decode: position of the current token; prefill: NULL
  // Q: q[((b*heads + h)*q_rows + s)*hd + e]
  f16* q;
  int q_rows;
  // K rows [s][hd] at k + b*k_bstride + kvh*k_hstride
  f16* k;
  size_t k_bstride, k_hstride;
  // V rows [s][hd] (KV cache layout), nullable
  f16* v;
  size_t v_bstride, v_hstride;
  // V transposed [hd][s] for prefill attention: vt + (b*kv_heads+kvh)*hd*vt_ld, nullable
  f16* vt;
  int vt_ld;
  float* tap;  // nullable [T, q+2kv] fp32 = Q_rope | K_rope | V
  FastDiv div_S, div_hd;  // by S and hd; set by prepare() on the host

  __host__ void prepare() {
    div_S = FastDiv((uint32_t)S);
    div_hd = FastDiv((uint32_t)hd);
  }
  HB_DEV void pos_of(int t, int& b, int& s) const {
    if (d_pos) {
      b = t;
      s = *d_pos;
    } else {
      b = div_S.div(t);
      s = t - b * S;
    }
  }
  // fb is the start of the 32-feature block that holds f0. The Q/K/V and head
  // boundaries are multiples of 32, so the region and the head follow from fb;
  // the prefill GEMM passes it as a wave-uniform value, which turns every
  // branch below into a scalar one.
  HB_DEV int region_start(int fb) const {
    return fb < q_dim ? 0 : fb < q_dim + kv_dim ? q_dim : q_dim + kv_dim;
  }
  // RoPE (cos, sin) of the feature pairs (f0, f0+1) and (f0+2, f0+3) of token
  // t; unused for V features.
  struct Aux {
    float2 c0, c1;
  };
  HB_DEV Aux load(int t, int f0, int fb) const {
    Aux a{};
    if (fb < q_dim + kv_dim) {
      int b, s;
      pos_of(t, b, s);
      const int fr = fb - region_start(fb);
      const int e = fr - div_hd.div(fr) * hd + (f0 - fb);
      const float2* rp = rope + (size_t)(e >> 1) * rope_ld + s;
      a.c0 = rp[0];
      a.c1 = rp[rope_ld];
    }
    return a;
  }
  HB_DEV void operator()(int t, int f0, f32x4 v4, const Aux& a, int fb) const {
    int b, s;
    pos_of(t, b, s);
    const int r0 = region_start(fb), fr = fb - r0;
    const int h = div_hd.div(fr), e = fr - h * hd + (f0 - fb);
    f32x4 o = v4;
    if (r0 < q_dim + kv_dim) {
      o.x = v4.x * a.c0.x - v4.y * a.c0.y;
      o.y = v4.y * a.c0.x + v4.x * a.c0.y;
      o.z = v4.z * a.c1.x - v4.w * a.c1.y;
      o.w = v4.w * a.c1.x + v4.z * a.c1.y;
    }
    f16x4 oh;
    oh.x = (f16)o.x;
    oh.y = (f16)o.y;
    oh.z = (f16)o.z;
    oh.w = (f16)o.w;
    // Q, K and V rows share one addressing form: base + b*bstride + h*hstride + s*hd + e
    f16* base;
    size_t bs, hs;
    int srow = s;
    if (r0 == 0) {
      base = q;
      hs = (size_t)q_rows * hd;
      bs = (size_t)heads * hs;
      if (d_pos) srow = 0;  // decode keeps one Q row per sequence
    } else if (r0 == q_dim) {
      base = k;
      bs = k_bstride;
      hs = k_hstride;
    } else {
      base = v;
      bs = v_bstride;
      hs = v_hstride;
    }
    if (base) *(f16x4*)(base + b * bs + h * hs + (size_t)srow * hd + e) = oh;
    if (r0 == q_dim + kv_dim && vt) {
      f16* p = vt + ((size_t)b * kv_heads + h) * hd * vt_ld + (size_t)e * vt_ld + s;
      p[0] = oh.x;
      p[vt_ld] = oh.y;
      p[2 * vt_ld] = oh.z;
      p[3 * vt_ld] = oh.w;
    }
    if (tap) *(f32x4*)(tap + (size_t)t * (q_dim + 2 * kv_dim) + f0) = o;
  }
  HB_DEV Aux load(int t, int f0) const { return load(t, f0, f0 & ~31); }
  HB_DEV void operator()(int t, int f0, f32x4 v4) const {
    (*this)(t, f0, v4, load(t, f0), f0 & ~31);
  }
};

}  // namespace hb
