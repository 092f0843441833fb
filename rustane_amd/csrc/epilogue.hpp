// GEMM epilogues. Both the prefill MFMA GEMM and the decode GEMV hand each
// lane's results to an epilogue as (token row t, first feature f0, 4 values
// for features f0..f0+3). f0 is always a multiple of 4, and feature blocks of
// 4 never straddle a Q/K/V or head boundary because hd % 64 == 0.
#pragma once
#include "common.hpp"

namespace hb {

// C[t, f0..f0+3] = v * scale (fp32). Plain GEMM output; scale undoes a
// power-of-two pre-scale of an fp16 operand (exact), 1 otherwise.
struct EpiStore {
  float* c;
  int ldc;
  float scale = 1.0f;
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    f32x4 o;
    o.x = v.x * scale;
    o.y = v.y * scale;
    o.z = v.z * scale;
    o.w = v.w * scale;
    *(f32x4*)(c + (size_t)t * ldc + f0) = o;
  }
};

// Split-K partial sums of the prefill GEMM: split blockIdx.y writes
// p[blockIdx.y * split_stride + t * ld + f0 ..]; splitk_reduce (gemm_launch.hpp) adds
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
// res may be the same buffer as out. One explicit fma per element: left to
// the compiler, whether v * alpha + r is fused differs between the kernel
// instances (tile shapes), and with it the result of a token row between
// batch sizes.
struct EpiResidual {
  const float* res;
  float* out;
  int ld;
  float alpha;
  using Aux = f32x4;
  HB_DEV f32x4 load(int t, int f0, int = 0) const { return *(const f32x4*)(res + (size_t)t * ld + f0); }
  HB_DEV void operator()(int t, int f0, f32x4 v, const f32x4& r, int = 0) const {
    f32x4 y;
    y.x = __builtin_fmaf(v.x, alpha, r.x);
    y.y = __builtin_fmaf(v.y, alpha, r.y);
    y.z = __builtin_fmaf(v.z, alpha, r.z);
    y.w = __builtin_fmaf(v.w, alpha, r.w);
    *(f32x4*)(out + (size_t)t * ld + f0) = y;
  }
  HB_DEV void operator()(int t, int f0, f32x4 v) const { (*this)(t, f0, v, load(t, f0)); }
};

// W1 and W3 are packed row-interleaved in groups of four: packed rows 4j..4j+3
// are W1 column 2j, W1 column 2j+1, W3 column 2j, W3 column 2j+1. A lane's
// 4 consecutive features are therefore (h1[u], h1[u+1], h3[u], h3[u+1]) with
// u = f0/2, and the SwiGLU gate (kernels/ffn_fused.rs:60-62) is formed in
// registers: gate = silu(h1) * h3.
// With split set, gate rows are split rows [T, 2*hidden] (hi | lo, common.hpp).
struct EpiSwiGLU {
  f16* gate;   // [T, hidden], or [T, 2*hidden] split
  float* tap;  // nullable [T, 2*hidden] = h1 | h3
  int hidden;
  bool split = false;
  // Decode with 8..16 sequences: gate in the decode GEMV's B-fragment order
  // (EpiSwiGLUFrag below); only gemv_swiglu reads this flag.
  bool frag = false;
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    const int u = f0 >> 1;
    const float g0 = silu_f(v.x) * v.z, g1 = silu_f(v.y) * v.w;
    f16x2 g;
    g.x = (f16)g0;
    g.y = (f16)g1;
    f16* row = gate + (size_t)t * (split ? 2 * hidden : hidden) + u;
    *(f16x2*)row = g;
    if (split) {
      f16x2 lo;
      lo.x = (f16)(g0 - (float)g.x);
      lo.y = (f16)(g1 - (float)g.y);
      *(f16x2*)(row + hidden) = lo;
    }
    if (tap) {
      float* r = tap + (size_t)t * 2 * hidden;
      r[u] = v.x;
      r[u + 1] = v.y;
      r[hidden + u] = v.z;
      r[hidden + u + 1] = v.w;
    }
  }
};

// The SwiGLU gate of EpiSwiGLU in the decode GEMV's B-fragment order over 16
// row slots: element (t, u) at ((u/32)*64 + t + 16*((u%32)/8))*8 + u%8, so
// the W2 GEMV reads each k-step's operand as one contiguous 1 KB block. A
// type of its own, so that the prefill GEMM's SwiGLU epilogue stays as it is.
struct EpiSwiGLUFrag {
  f16* gate;
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    const int u = f0 >> 1;
    f16x2 g;
    g.x = (f16)(silu_f(v.x) * v.z);
    g.y = (f16)(silu_f(v.y) * v.w);
    *(f16x2*)(gate + ((size_t)(u >> 5) * 64 + t + 16 * ((u & 31) >> 3)) * 8 + (u & 7)) = g;
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
//
// EpiQKV holds the parameters; the kernels run EpiQKVAt<DECODE, MODE>, which
// fixes at compile time whether the position comes from d_pos (decode) or
// from the token index (prefill), and which outputs exist (mode()): the
// optional low parts and tap, tested per quad, cost the 7B QKV epilogue
// ~4 us and the 5B one at 2048 tokens ~8 us when they are runtime branches. A runtime d_pos test in the prefill GEMM left a load
// on one side of a branch in every quad, and the wait it needs at the join
// (vmcnt(0) on gfx950, where stores count too) serialised every quad's stores
// behind the previous ones: 7B QKV epilogue 9.5 us, 5B at 2048 tokens 39 us.
struct EpiQKV {
  int q_dim, kv_dim, hd, S, heads, kv_heads;
  const float4* rope;  // [hd/4][rope_ld] (cos, sin of pair 2q, cos, sin of pair 2q+1)
  int rope_ld;         // positions per row
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
  // Low parts of the two-term fp16 form (common.hpp) in the same layouts as
  // q, k, v and vt; all NULL for plain fp16 outputs.
  f16 *q_lo = nullptr, *k_lo = nullptr, *v_lo = nullptr, *vt_lo = nullptr;
  FastDiv div_S, div_hd;  // by S and hd; set by prepare() on the host

  __host__ void prepare() {
    div_S = FastDiv((uint32_t)S);
    div_hd = FastDiv((uint32_t)hd);
  }
  template <bool DEC>
  HB_DEV void pos_of(int t, int& b, int& s) const {
    if constexpr (DEC) {
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
  template <bool DEC>
  HB_DEV Aux load_at(int t, int f0, int fb) const {
    Aux a{};
    if (fb < q_dim + kv_dim) {
      int b, s;
      pos_of<DEC>(t, b, s);
      const int fr = fb - region_start(fb);
      const int e = fr - div_hd.div(fr) * hd + (f0 - fb);
      const float4 r = rope[(size_t)(e >> 2) * rope_ld + s];  // e % 4 == 0
      a.c0 = make_float2(r.x, r.y);
      a.c1 = make_float2(r.z, r.w);
    }
    return a;
  }
  // Output modes of the kernels' instances (EpiQKVAt): PLAIN writes fp16 Q,
  // K and V^T and/or V rows (every layer but the two-term ones); SPLIT also
  // writes the low parts (q_lo .. vt_lo); FULL also the fp32 tap.
  enum Mode { PLAIN = 0, SPLIT = 1, FULL = 2 };
  __host__ int mode() const {
    return tap ? FULL : (q_lo || k_lo || v_lo || vt_lo) ? SPLIT : PLAIN;
  }
  template <bool DEC, int MODE>
  HB_DEV void store_at(int t, int f0, f32x4 v4, const Aux& a, int fb) const {
    int b, s;
    pos_of<DEC>(t, b, s);
    const int r0 = region_start(fb), fr = fb - r0;
    const int h = div_hd.div(fr), e = fr - h * hd + (f0 - fb);
    f32x4 o = v4;
    if (r0 < q_dim + kv_dim) {
      // Contraction is left to the compiler here: explicit fma forms, and
      // contract(off), make the 256x256 instances spill 620-660 bytes to
      // scratch. The fusion it picks is the same in every prefill tile shape
      // (a batch row equals its sequence run alone, bit for bit, tested).
      o.x = v4.x * a.c0.x - v4.y * a.c0.y;
      o.y = v4.y * a.c0.x + v4.x * a.c0.y;
      o.z = v4.z * a.c1.x - v4.w * a.c1.y;
      o.w = v4.w * a.c1.x + v4.z * a.c1.y;
    }
    const f16x4 oh = f16x4_hi(o);
    if constexpr (MODE == PLAIN) {
      // one f16x4 store per quad (Q, K or V rows) and, for V^T, four
      // 2-byte stores; every branch is wave-uniform (fb)
      if (r0 == 0) {
        const size_t hs = (size_t)q_rows * hd;
        *(f16x4*)(q + b * (heads * hs) + h * hs + (size_t)(DEC ? 0 : s) * hd + e) = oh;
      } else if (r0 == q_dim) {
        *(f16x4*)(k + b * k_bstride + h * k_hstride + (size_t)s * hd + e) = oh;
      } else {
        if (v) *(f16x4*)(v + b * v_bstride + h * v_hstride + (size_t)s * hd + e) = oh;
        if (vt) {
          f16* p = vt + ((size_t)b * kv_heads + h) * hd * vt_ld + (size_t)e * vt_ld + s;
          p[0] = oh.x;
          p[vt_ld] = oh.y;
          p[2 * vt_ld] = oh.z;
          p[3 * vt_ld] = oh.w;
        }
      }
      return;
    }
    // Q, K and V rows share one addressing form: base + b*bstride + h*hstride + s*hd + e
    f16 *base, *base_lo;
    size_t bs, hs;
    int srow = s;
    if (r0 == 0) {
      base = q;
      base_lo = q_lo;
      hs = (size_t)q_rows * hd;
      bs = (size_t)heads * hs;
      if (DEC) srow = 0;  // decode keeps one Q row per sequence
    } else if (r0 == q_dim) {
      base = k;
      base_lo = k_lo;
      bs = k_bstride;
      hs = k_hstride;
    } else {
      base = v;
      base_lo = v_lo;
      bs = v_bstride;
      hs = v_hstride;
    }
    const size_t off = b * bs + h * hs + (size_t)srow * hd + e;
    if (base) *(f16x4*)(base + off) = oh;
    const bool lo = base_lo || (r0 == q_dim + kv_dim && vt_lo);
    const f16x4 ol = lo ? f16x4_lo(o, oh) : f16x4{};
    if (base_lo) *(f16x4*)(base_lo + off) = ol;
    if (r0 == q_dim + kv_dim && vt) {
      const size_t vo = ((size_t)b * kv_heads + h) * hd * vt_ld + (size_t)e * vt_ld + s;
      f16* p = vt + vo;
      p[0] = oh.x;
      p[vt_ld] = oh.y;
      p[2 * vt_ld] = oh.z;
      p[3 * vt_ld] = oh.w;
      if (vt_lo) {
        f16* pl = vt_lo + vo;
        pl[0] = ol.x;
        pl[vt_ld] = ol.y;
        pl[2 * vt_ld] = ol.z;
        pl[3 * vt_ld] = ol.w;
      }
    }
    if (tap) *(f32x4*)(tap + (size_t)t * (q_dim + 2 * kv_dim) + f0) = o;
  }
};

template <bool DECODE, int MODE>
struct EpiQKVAt : EpiQKV {
  EpiQKVAt() = default;
  __host__ explicit EpiQKVAt(const EpiQKV& e) : EpiQKV(e) {}
  HB_DEV Aux load(int t, int f0, int fb) const { return load_at<DECODE>(t, f0, fb); }
  // Prefill tiles stage the RoPE rows of their TT tokens into LDS (the
  // GEMM's EpiStage): table entry q of token t0 + j goes to lo[q * TT + j]
  // for q < hd/8 and to hi[(q - hd/8) * TT + j] above. Thread tid keeps
  // token j = tid % TT (one position) and copies rows q = tid / TT,
  // + NT/TT, ... in batches of 8 loads; tiles of V features only need none.
  static constexpr bool kStage = !DECODE;
  template <int TT, int NT>
  HB_DEV void stage(float4* lo, float4* hi, int t0, int f_base, int tid) const {
    static_assert(NT % TT == 0, "whole tokens per thread pass");
    if (f_base >= q_dim + kv_dim) return;  // uniform over the workgroup
    constexpr int QS = NT / TT;  // rows per pass
    const int j = tid % TT, nq = hd >> 2, half = hd >> 3;
    int b, s;
    pos_of<false>(t0 + j, b, s);  // a token past T still maps into [0, S)
    const float4* src = rope + s;
    for (int q0 = tid / TT; q0 < nq; q0 += 8 * QS) {
      float4 r0, r1, r2, r3, r4, r5, r6, r7;
      auto ld = [&](int k, float4& r) {
        if (q0 + k * QS < nq) r = src[(size_t)(q0 + k * QS) * rope_ld];
      };
      auto st = [&](int k, const float4& r) {
        const int q = q0 + k * QS;
        if (q < nq) (q < half ? lo + q * TT : hi + (q - half) * TT)[j] = r;
      };
      ld(0, r0), ld(1, r1), ld(2, r2), ld(3, r3), ld(4, r4), ld(5, r5), ld(6, r6), ld(7, r7);
      st(0, r0), st(1, r1), st(2, r2), st(3, r3), st(4, r4), st(5, r5), st(6, r6), st(7, r7);
    }
  }
  // load_at from the staged rows, token t0 + j
  HB_DEV Aux load_staged(const float4* lo, const float4* hi, int j, int tt, int f0, int fb) const {
    Aux a{};
    if (fb < q_dim + kv_dim) {
      const int fr = fb - region_start(fb);
      const int e = fr - div_hd.div(fr) * hd + (f0 - fb), q = e >> 2, half = hd >> 3;
      // the 8 rows of one accumulator row's quads start at a multiple of 8:
      // the half is wave-uniform
      const float4 r = (q < half ? lo + q * tt : hi + (q - half) * tt)[j];
      a.c0 = make_float2(r.x, r.y);
      a.c1 = make_float2(r.z, r.w);
    }
    return a;
  }
  HB_DEV void operator()(int t, int f0, f32x4 v4, const Aux& a, int fb) const {
    store_at<DECODE, MODE>(t, f0, v4, a, fb);
  }
  // Prefill PLAIN through the GEMM's EpiRows: (b, s) once per token, the
  // row pointer of (Q/K/V region, head, b, s) once per 32-feature block and
  // token, then per quad only the feature offset -- the same stores as
  // store_at without its per-quad division and 64-bit address arithmetic
  // (QKV GEMM at 512 tokens in the forward 68.8 -> 66.9 us on one box).
  static constexpr bool kRows = !DECODE && MODE == PLAIN;
  struct Tok {
    int b, s;
  };
  struct Row {
    f16* p;   // row (b, s) of head h in the block's region (Q, K or V), at feature 0
    f16* pt;  // column s of head h in V^T (V region)
    int e0;   // feature of fb within its head
  };
  HB_DEV Tok tok(int t) const {
    Tok r;
    pos_of<false>(t, r.b, r.s);
    return r;
  }
  HB_DEV Row row(const Tok& tk, int fb) const {
    const int r0 = region_start(fb), fr = fb - r0, h = div_hd.div(fr);
    Row r{nullptr, nullptr, fr - h * hd};
    if (r0 == 0) {
      r.p = q + ((size_t)tk.b * heads + h) * q_rows * hd + (size_t)tk.s * hd;
    } else if (r0 == q_dim) {
      r.p = k + tk.b * k_bstride + h * k_hstride + (size_t)tk.s * hd;
    } else {
      if (v) r.p = v + tk.b * v_bstride + h * v_hstride + (size_t)tk.s * hd;
      if (vt) r.pt = vt + ((size_t)tk.b * kv_heads + h) * hd * vt_ld + tk.s;
    }
    return r;
  }
  HB_DEV void store_row(const Row& r, int f0, f32x4 v4, const Aux& a, int fb) const {
    const int r0 = region_start(fb), e = r.e0 + (f0 - fb);
    f32x4 o = v4;
    if (r0 < q_dim + kv_dim) {  // as store_at
      o.x = v4.x * a.c0.x - v4.y * a.c0.y;
      o.y = v4.y * a.c0.x + v4.x * a.c0.y;
      o.z = v4.z * a.c1.x - v4.w * a.c1.y;
      o.w = v4.w * a.c1.x + v4.z * a.c1.y;
    }
    const f16x4 oh = f16x4_hi(o);
    if (r0 < q_dim + kv_dim || v) *(f16x4*)(r.p + e) = oh;
    if (r0 == q_dim + kv_dim && vt) {
      f16* p = r.pt + (size_t)e * vt_ld;
      p[0] = oh.x;
      p[vt_ld] = oh.y;
      p[2 * vt_ld] = oh.z;
      p[3 * vt_ld] = oh.w;
    }
  }
  HB_DEV Aux load(int t, int f0) const { return load(t, f0, f0 & ~31); }
  HB_DEV void operator()(int t, int f0, f32x4 v4) const { (*this)(t, f0, v4, load(t, f0), f0 & ~31); }
};

// ---- training (backward) epilogues ----

// g[t * ld + f0 ..] += v: weight-gradient accumulation into the fp32 gradient
// arena (layer.rs:1864-1867 accumulate_dw: dW += A B^T). Each element belongs
// to exactly one lane of one tile, so the read-modify-write needs no atomics.
// The old values are Aux operands, so the prefill GEMM loads them one
// accumulator row ahead of the stores (as for EpiResidual) instead of exposing
// a load latency per quad.
struct EpiAccum {
  float* g;
  int ld;
  float scale = 1.0f;  // as EpiStore
  using Aux = f32x4;
  HB_DEV f32x4 load(int t, int f0, int = 0) const { return *(const f32x4*)(g + (size_t)t * ld + f0); }
  HB_DEV void operator()(int t, int f0, f32x4 v, const f32x4& a, int = 0) const {
    f32x4 o;
    o.x = a.x + v.x * scale;
    o.y = a.y + v.y * scale;
    o.z = a.z + v.z * scale;
    o.w = a.w + v.w * scale;
    *(f32x4*)(g + (size_t)t * ld + f0) = o;
  }
  HB_DEV void operator()(int t, int f0, f32x4 v) const { (*this)(t, f0, v, load(t, f0)); }
};

// The same two with the sum of squares of the stored values returned to the
// GEMM, which writes one total per output tile to sq_out (the gradient norm's
// partial sums, taken while the gradient is written instead of by a second
// pass over the arena).
struct EpiStoreSq {
  static constexpr bool kSumSq = true;
  float* c;
  int ldc;
  float scale;
  float* sq_out;
  HB_DEV float operator()(int t, int f0, f32x4 v) const {
    f32x4 o;
    o.x = v.x * scale;
    o.y = v.y * scale;
    o.z = v.z * scale;
    o.w = v.w * scale;
    *(f32x4*)(c + (size_t)t * ldc + f0) = o;
    return o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
  }
};
struct EpiAccumSq {
  static constexpr bool kSumSq = true;
  float* g;
  int ld;
  float scale;
  float* sq_out;
  using Aux = f32x4;
  HB_DEV f32x4 load(int t, int f0, int = 0) const { return *(const f32x4*)(g + (size_t)t * ld + f0); }
  HB_DEV float operator()(int t, int f0, f32x4 v, const f32x4& a, int = 0) const {
    f32x4 o;
    o.x = a.x + v.x * scale;
    o.y = a.y + v.y * scale;
    o.z = a.z + v.z * scale;
    o.w = a.w + v.w * scale;
    *(f32x4*)(g + (size_t)t * ld + f0) = o;
    return o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
  }
  HB_DEV float operator()(int t, int f0, f32x4 v) const { return (*this)(t, f0, v, load(t, f0)); }
};

// SwiGLU backward (layer.rs:1657-1666, cpu/silu.rs:20-33): v = dgate of hidden
// units u..u+3 of token t; with h1, h3 the forward pre-activations (tap [T][2h]
// = h1 | h3) and sig = 1/(1+exp(-h1)):
//   dh3 = dgate * h1 sig,   dh1 = dgate * h3 * sig (1 + h1 (1 - sig)).
// The result is written token-major (dh [T][2h], input of dX = dH W13) in the
// packed W1|W3 row order (see EpiSwiGLU): eight consecutive halfs dh1[u],
// dh1[u+1], dh3[u], dh3[u+1], dh1[u+2], dh1[u+3], dh3[u+2], dh3[u+3], one
// 16-byte store. (Its feature-major copy for dW13 is made by a separate
// 16-byte-access transpose: eight 2-byte scatters per lane here cost more.)
struct EpiSiluBwd {
  const float* tap;  // [T][2h] = h1 | h3
  f16* dh;           // [T][2h]
  int hidden;
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    const float* r = tap + (size_t)t * 2 * hidden;
    const f32x4 h1 = *(const f32x4*)(r + f0), h3 = *(const f32x4*)(r + hidden + f0);
    const float g[4] = {v.x, v.y, v.z, v.w}, a[4] = {h1.x, h1.y, h1.z, h1.w},
                b[4] = {h3.x, h3.y, h3.z, h3.w};
    float d1[4], d3[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sg = 1.0f / (1.0f + __expf(-a[i]));
      d3[i] = g[i] * (a[i] * sg);
      d1[i] = g[i] * b[i] * (sg * (1.0f + a[i] * (1.0f - sg)));
    }
    const float o[8] = {d1[0], d1[1], d3[0], d3[1], d1[2], d1[3], d3[2], d3[3]};
    f16x8 h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (f16)o[i];
    *(f16x8*)(dh + (size_t)t * 2 * hidden + 2 * f0) = h;
  }
};

// Token-major [B*S][H*hd] result stored head-major as fp16: out[((b*H + h) *
// rows + s) * hd + e] for token t = b*S + s (attention-output gradient, read
// per head by the attention backward products).
struct EpiHeads {
  f16* out;
  int S, H, hd, rows;
  HB_DEV void operator()(int t, int f0, f32x4 v) const {
    const int b = t / S, s = t - b * S, h = f0 / hd, e = f0 - h * hd;
    f16x4 o;
    o.x = (f16)v.x;
    o.y = (f16)v.y;
    o.z = (f16)v.z;
    o.w = (f16)v.w;
    *(f16x4*)(out + (((size_t)b * H + h) * rows + s) * hd + e) = o;
  }
};

}  // namespace hb
