// C ABI of libhip_bridge.so (declared in include/hip_bridge.h): contexts, the
// device model, the prefill forward, the per-kernel entry points and the decode
// loop. Host orchestration only; kernels live in gemm*.hip, gemv.hip,
// attention.hip and elementwise.hip.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/hip_bridge.h"
#include "internal.hpp"
#include "synth.hpp"

using namespace hb;

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
static thread_local std::string g_err;
static std::atomic<int> g_inject{0};

static int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HB_INJECT_CHECK()                                                  \
  do {                                                                     \
    if (int c_ = g_inject.load()) return fail(HB_E_INJECTED, "injected error %d", c_); \
  } while (0)

#define HIP_TRY(expr)                                                                    \
  do {                                                                                   \
    hipError_t e_ = (expr);                                                              \
    if (e_ != hipSuccess)                                                                \
      return fail(e_ == hipErrorOutOfMemory ? HB_E_OOM : HB_E_DEVICE, "%s failed: %s (%s:%d)", \
                  #expr, hipGetErrorString(e_), __FILE__, __LINE__);                     \
  } while (0)

#define TRY(expr)                \
  do {                           \
    int r_ = (expr);             \
    if (r_ != HB_OK) return r_;  \
  } while (0)

// ---------------------------------------------------------------------------
// objects
// ---------------------------------------------------------------------------
struct hb_ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t user = nullptr;
  hipStream_t capture = nullptr;
  int* d_err = nullptr;
  hipStream_t stream() const { return user ? user : own; }
};

namespace {

struct LayerW {
  f16* wqkv = nullptr;  // [q+2kv, dim]
  f16* wo = nullptr;    // [dim, q]
  f16* w13 = nullptr;   // [2*hidden, dim], row-interleaved (see EpiSwiGLU)
  f16* w2 = nullptr;    // [dim, hidden]
  float* g1 = nullptr;
  float* g2 = nullptr;
  bool uploaded = false;
  // decode copies of the four matrices in fragment-tiled order (gemv.hip)
  f16 *t_wqkv = nullptr, *t_wo = nullptr, *t_w13 = nullptr, *t_w2 = nullptr;
};

// Prefill activations. Q/K/V^T rows are padded per sequence to S_pad (multiple
// of 32) for the attention kernel.
struct Workspace {
  long cap_T = 0, cap_Tpad = 0;
  void* base = nullptr;
  float *x = nullptr, *x2 = nullptr, *logits = nullptr, *loss = nullptr, *mean = nullptr;
  f16 *xn = nullptr, *q = nullptr, *k = nullptr, *vt = nullptr, *attn = nullptr, *gate = nullptr;
  uint32_t *tok = nullptr, *tgt = nullptr;
  // split-operand layers (hb_model::precise_layers): xn, attn and gate have
  // room for split rows [T, 2K], and Q, K, V^T have low parts
  bool split = false;
  f16 *q_lo = nullptr, *k_lo = nullptr, *vt_lo = nullptr;
};

}  // namespace


namespace hb {
struct TrainState;
}  // namespace hb

struct hb_model {
  hb_ctx* ctx = nullptr;
  int device = 0;
  hb_model_config cfg{};
  void* wbase = nullptr;
  size_t wbytes = 0;
  std::vector<LayerW> layers;
  f16* embed = nullptr;  // [vocab, dim]
  float* gamma_f = nullptr;
  bool embed_uploaded = false;
  float4* rope = nullptr;  // RoPE table, [hd/4][rope_len] (ensure_rope)
  int rope_len = 0;
  float* staging = nullptr;
  size_t staging_floats = 0;
  Workspace ws;
  int graph_epoch = 0;  // bumped when a captured decode graph goes stale
  // Decode copy of every matrix (fragment-tiled), allocated on first decode
  // use and rebuilt from the row-major weights after any upload.
  void* dbase = nullptr;
  size_t dbytes = 0;
  f16* t_embed = nullptr;
  bool dec_stale = true;
  // split-K partial sums of the prefill residual GEMMs (gemm_splits)
  float* splitk = nullptr;
  size_t splitk_floats = 0;
  // Training state (transposed weights, kept activations, backward scratch),
  // allocated by the first hb_forward_backward; wt_stale marks the transposed
  // weights out of date after any weight write.
  TrainState* train = nullptr;
  bool wt_stale = true;
  // Forward of one launch sequence replayed from a HIP graph: after a first
  // eager run of a call shape (fwd_seen), the next identical call captures
  // it (fwd_exec); later identical calls replay it with one launch.
  struct FwdKey {
    int B = 0, S = 0, np = -1, epoch = -1;
    float softcap = 0.f;
    const void *tok = nullptr, *tgt = nullptr, *loss = nullptr, *logits = nullptr, *mean = nullptr;
    const void *ws = nullptr, *splitk = nullptr;
    bool operator==(const FwdKey& o) const {
      return B == o.B && S == o.S && np == o.np && epoch == o.epoch && softcap == o.softcap &&
             tok == o.tok && tgt == o.tgt && loss == o.loss && logits == o.logits && mean == o.mean &&
             ws == o.ws && splitk == o.splitk;
    }
  };
  FwdKey fwd_seen, fwd_key;
  hipGraph_t fwd_graph = nullptr;
  hipGraphExec_t fwd_exec = nullptr;
  // The first precise_layers layers of a prefill or decode forward run on
  // two-term fp16 operands (common.hpp): their GEMM/GEMV inputs, Q, K, V and
  // attention probabilities carry ~22 bits instead of fp16's 11. Rounding in
  // the first layer, where the residual stream is still the small embedding,
  // sets most of the deep models' distance from fp32 arithmetic.
  int precise_layers = 1;
};

namespace hb {

inline long round64(long v) { return (v + 63) & ~63L; }

// Activations of one layer that the backward reads (the reference's per-layer
// forward cache, layer.rs:684-806 with `cache`): token-major [T, features]
// except Q/K/V, which are head-major [B][heads][Sp][hd] with Sp = S rounded up
// to 64 (zero padding rows).
struct LayerAct {
  float *x, *x2, *h13;  // layer input, attention residual, FFN pre-activations h1|h3
  f16 *xn, *x2n, *q, *k, *v, *attn, *gate;
  float* lse;  // [B][heads][Sp] attention log-sum-exp (log2 units) for the fused backward
};

struct TrainState {
  // transposed fp16 weights for the dX products
  void* wtbase = nullptr;
  std::vector<f16*> wqkvT, woT, w13T, w2T;  // [dim][qkv], [q][dim], [dim][2h], [h][dim]
  f16* eT = nullptr;                        // [dim][Vp], columns >= vocab zero
  // activations and backward scratch for one (B, S)
  void* abase = nullptr;
  size_t abytes = 0;
  int B = 0, S = 0;
  std::vector<LayerAct> act;
  float *xL = nullptr, *logits = nullptr, *loss = nullptr, *mean = nullptr;
  f16* xf = nullptr;
  uint32_t *tok = nullptr, *tgt = nullptr;
  float *dy = nullptr, *dx2 = nullptr, *dtmp = nullptr, *rinv = nullptr, *part = nullptr;
  float* Drow = nullptr;  // [B][heads][Sp] rowsum(P * dP) of the attention backward
  f16 *d16 = nullptr, *d16T = nullptr, *dh = nullptr, *dhT = nullptr, *actT = nullptr;
  f16 *dqkv = nullptr, *dqkvT = nullptr, *dl = nullptr, *dlT = nullptr;
  f16 *dA = nullptr, *dAT = nullptr, *qT = nullptr, *kT = nullptr, *vt = nullptr;
  // hb_train_forward left its activations for hb_train_backward (the
  // reference's ForwardResult.caches); any other training call clears it.
  bool kept = false;
  // The softcap the kept logits were computed with: the backward's
  // derivative must use it even if hb_model_set_softcap (or an inference
  // forward with another softcap) ran in between.
  float softcap = 0.f;
  // device staging of ForwardResult's host views, grown on demand
  float* views = nullptr;
  size_t views_floats = 0;
};

void train_free(TrainState* t) {
  if (!t) return;
  if (t->wtbase) (void)hipFree(t->wtbase);
  if (t->abase) (void)hipFree(t->abase);
  if (t->views) (void)hipFree(t->views);
  delete t;
}

}  // namespace hb

struct hb_kv {
  hb_model* model = nullptr;
  int device = 0;
  int B = 0, ctx_max = 0, ctx_cap = 0, nch = 0;
  int len = 0;
  f16* cache = nullptr;  // [L][B][2][KVH][ctx_cap][hd]
  size_t cache_bytes = 0;
  void* sbase = nullptr;  // small decode buffers
  int *d_pos = nullptr, *d_pos0 = nullptr;
  uint32_t *d_tok = nullptr, *d_next = nullptr, *d_hist = nullptr;
  float *x = nullptr, *x2 = nullptr, *logits = nullptr, *part_o = nullptr, *part_ml = nullptr;
  bool attn_in_wo = false;       // chunk partials combined by the Wo GEMV
  float* amax_val = nullptr;  // greedy argmax partials [B][vocab/16]
  int* amax_idx = nullptr;
  f16 *xn = nullptr, *qd = nullptr, *attn = nullptr, *gate = nullptr;
  // Layers l < np run on two-term fp16 operands (hb_model::precise_layers at
  // creation): their K/V low parts live in lo_cache [np][B][K,V][KVH][ctx_cap][hd],
  // the query's in qd_lo; xn, attn and gate have room for split rows.
  int np = 0;
  f16* lo_cache = nullptr;
  size_t lo_bytes = 0;
  f16* qd_lo = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int graph_epoch = -1;
};

namespace {

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

int check_err_word(hb_ctx* ctx) {
  int h = 0;
  HIP_TRY(hipMemcpyAsync(&h, ctx->d_err, sizeof(int), hipMemcpyDeviceToHost, ctx->stream()));
  HIP_TRY(hipStreamSynchronize(ctx->stream()));
  if (h) {
    int zero = 0;
    HIP_TRY(hipMemcpyAsync(ctx->d_err, &zero, sizeof(int), hipMemcpyHostToDevice, ctx->stream()));
    HIP_TRY(hipStreamSynchronize(ctx->stream()));
    return fail(HB_E_INVALID, "device saw an out-of-range %s id (error word 0x%x)",
                (h & 1) ? "token" : "target", h);
  }
  return HB_OK;
}

float alpha_of(const hb_model_config& c) { return c.residual_alpha; }

int validate_config(const hb_model_config& c) {
  if (c.dim <= 0 || c.hidden <= 0 || c.heads <= 0 || c.kv_heads <= 0 || c.hd <= 0 || c.seq <= 0 ||
      c.nlayers <= 0 || c.vocab <= 0)
    return fail(HB_E_CONFIG, "all dimensions must be positive");
  if (c.hd != 64 && c.hd != 128) return fail(HB_E_CONFIG, "hd must be 64 or 128 (got %d)", c.hd);
  if (c.q_dim != c.heads * c.hd) return fail(HB_E_CONFIG, "q_dim != heads*hd");
  if (c.kv_dim != c.kv_heads * c.hd) return fail(HB_E_CONFIG, "kv_dim != kv_heads*hd");
  if (c.heads % c.kv_heads) return fail(HB_E_CONFIG, "heads %% kv_heads != 0");
  if (c.gqa_ratio != c.heads / c.kv_heads) return fail(HB_E_CONFIG, "gqa_ratio != heads/kv_heads");
  if (c.dim % 64 || c.hidden % 64 || c.q_dim % 64 || c.kv_dim % 64 || c.vocab % 64)
    return fail(HB_E_CONFIG, "dim, hidden, q_dim, kv_dim and vocab must be multiples of 64");
  if (c.vocab >= (1 << 30) || c.dim > 65536 || c.hidden > 262144)
    return fail(HB_E_CONFIG, "dimension too large");
  return HB_OK;
}

// RoPE table exactly as kernels/sdpa_fwd.rs:18-33 computes it:
// theta = p / base^(2i/hd) in f32; (cos, sin) per (i, p), stored pair-major
// [hd/4][len] of float4 (cos, sin of pair 2q, cos, sin of pair 2q + 1): one
// 16-byte load gives a lane the rotation of its 4 consecutive features, and
// consecutive positions are adjacent (the prefill GEMM epilogue reads one
// entry for 32 consecutive tokens at a time).
int ensure_rope(hb_model* m, int len) {
  if (len <= m->rope_len) return HB_OK;
  const int half = m->cfg.hd / 2;
  std::vector<float> tab((size_t)len * half * 2);
  for (int p = 0; p < len; ++p)
    for (int i = 0; i < half; ++i) {
      const float theta =
          (float)p / powf(m->cfg.rope_theta, 2.0f * (float)i / (float)m->cfg.hd);
      float* t = &tab[(((size_t)(i >> 1) * len + p) * 2 + (i & 1)) * 2];
      t[0] = cosf(theta);
      t[1] = sinf(theta);
    }
  HIP_TRY(hipStreamSynchronize(m->ctx->stream()));
  if (m->rope) HIP_TRY(hipFree(m->rope));
  m->rope = nullptr;
  HIP_TRY(hipMalloc(&m->rope, tab.size() * sizeof(float)));
  HIP_TRY(hipMemcpy(m->rope, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice));
  m->rope_len = len;
  m->graph_epoch++;  // captured decode graphs hold the old table address
  return HB_OK;
}

int ensure_staging(hb_model* m, size_t floats) {
  if (floats <= m->staging_floats) return HB_OK;
  HIP_TRY(hipStreamSynchronize(m->ctx->stream()));
  if (m->staging) HIP_TRY(hipFree(m->staging));
  m->staging = nullptr;
  HIP_TRY(hipMalloc(&m->staging, floats * sizeof(float)));
  m->staging_floats = floats;
  return HB_OK;
}

// True while the context's current stream is being captured into a graph:
// nothing may allocate, free or synchronise then.
bool capturing(hb_model* m) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(m->ctx->stream(), &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

int ensure_workspace(hb_model* m, long T, long Tpad, bool need_split = false) {
  Workspace& w = m->ws;
  const bool split = need_split || m->precise_layers > 0 || w.split;
  if (T <= w.cap_T && Tpad <= w.cap_Tpad && w.split == split) return HB_OK;
  if (capturing(m)) return fail(HB_E_STATE, "the workspace must grow to %ld tokens while the stream is captured", T);
  T = std::max(T, w.cap_T);
  Tpad = std::max(Tpad, w.cap_Tpad);
  const hb_model_config& c = m->cfg;
  HIP_TRY(hipStreamSynchronize(m->ctx->stream()));
  if (w.base) HIP_TRY(hipFree(w.base));
  w = Workspace{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += align256(bytes);
    return o;
  };
  const size_t sf = split ? 2 : 1;  // split rows take twice the halves
  const size_t o_x = take(T * c.dim * 4), o_x2 = take(T * c.dim * 4);
  const size_t o_logits = take((size_t)T * c.vocab * 4), o_loss = take(T * 4), o_mean = take(4);
  const size_t o_xn = take(sf * T * c.dim * 2), o_attn = take(sf * T * c.q_dim * 2);
  const size_t o_gate = take(sf * (size_t)T * c.hidden * 2);
  const size_t o_q = take(Tpad * c.q_dim * 2), o_k = take(Tpad * c.kv_dim * 2);
  const size_t o_vt = take(Tpad * c.kv_dim * 2);
  const size_t o_tok = take(T * 4), o_tgt = take(T * 4);
  const size_t o_qlo = split ? take(Tpad * c.q_dim * 2) : 0, o_klo = split ? take(Tpad * c.kv_dim * 2) : 0;
  const size_t o_vtlo = split ? take(Tpad * c.kv_dim * 2) : 0;
  char* base = nullptr;
  HIP_TRY(hipMalloc(&base, off));
  w.base = base;
  w.cap_T = T;
  w.cap_Tpad = Tpad;
  w.split = split;
  if (split) {
    w.q_lo = (f16*)(base + o_qlo);
    w.k_lo = (f16*)(base + o_klo);
    w.vt_lo = (f16*)(base + o_vtlo);
  }
  w.x = (float*)(base + o_x);
  w.x2 = (float*)(base + o_x2);
  w.logits = (float*)(base + o_logits);
  w.loss = (float*)(base + o_loss);
  w.mean = (float*)(base + o_mean);
  w.xn = (f16*)(base + o_xn);
  w.attn = (f16*)(base + o_attn);
  w.gate = (f16*)(base + o_gate);
  w.q = (f16*)(base + o_q);
  w.k = (f16*)(base + o_k);
  w.vt = (f16*)(base + o_vt);
  w.tok = (uint32_t*)(base + o_tok);
  w.tgt = (uint32_t*)(base + o_tgt);
  // Padding rows/columns of Q, K and V^T are read (and masked) by attention:
  // keep them finite.
  hipStream_t st = m->ctx->stream();
  HIP_TRY(fill_f16_zero(w.q, (size_t)Tpad * c.q_dim, st));
  HIP_TRY(fill_f16_zero(w.k, (size_t)Tpad * c.kv_dim, st));
  HIP_TRY(fill_f16_zero(w.vt, (size_t)Tpad * c.kv_dim, st));
  if (split) {
    HIP_TRY(fill_f16_zero(w.q_lo, (size_t)Tpad * c.q_dim, st));
    HIP_TRY(fill_f16_zero(w.k_lo, (size_t)Tpad * c.kv_dim, st));
    HIP_TRY(fill_f16_zero(w.vt_lo, (size_t)Tpad * c.kv_dim, st));
  }
  return HB_OK;
}

int S_pad_of(int S) { return (S + 31) & ~31; }

// The forward kernels index activations with 32-bit element offsets (row x K
// in the GEMM loads, row x vocab in the logits and loss kernels, token x
// q_dim in attention) and launch one grid layer per sequence. Rejects B x S
// token counts whose largest activation, rounded up to the GEMM's 64-row
// tile, would not fit, before anything is allocated or launched.
int check_token_count(const hb_model_config& c, long B, long S) {
  const long T = B * S, Tp = B * S_pad_of((int)std::min<long>(S, 1L << 30));
  const long widest = std::max({(long)c.vocab, 2L * c.hidden, (long)c.q_dim + 2L * c.kv_dim, (long)c.dim});
  if (B > 65535 || round64(T) * widest >= (1L << 31) || round64(Tp) * (long)c.q_dim >= (1L << 31))
    return fail(HB_E_INVALID, "B=%ld S=%ld: %ld tokens x %ld features exceeds the 2^31-element activation limit",
                B, S, T, widest);
  return HB_OK;
}

// Scratch for a residual GEMM of this shape: grown on demand, empty when the
// shape does not split. A captured forward (forward_device_impl) reserves it
// before the capture starts; growing it during a capture is refused
// (HB_E_STATE), since it would allocate and synchronise inside the graph.
int residual_scratch(hb_model* m, int N, int T, int K, GemmScratch& out, int wgs = 256) {
  out = GemmScratch{m->splitk, m->splitk_floats, wgs};
  bool wide;
  const int S = std::max(gemm_splits(N, T, K, wgs), gemm_norm_splits(N, T, K, wgs, &wide));
  if (S <= 1) return HB_OK;
  const size_t need = (size_t)S * T * N;
  if (need > m->splitk_floats) {
    if (capturing(m))
      return fail(HB_E_STATE, "split-K scratch must grow to %zu floats while the stream is captured", need);
    HIP_TRY(hipStreamSynchronize(m->ctx->stream()));
    if (m->splitk) HIP_TRY(hipFree(m->splitk));
    m->splitk = nullptr;
    m->splitk_floats = 0;
    HIP_TRY(hipMalloc(&m->splitk, need * 4));
    m->splitk_floats = need;
  }
  out = GemmScratch{m->splitk, m->splitk_floats, wgs};
  return HB_OK;
}

bool weights_ready(hb_model* m) {
  if (!m->embed_uploaded) return false;
  for (auto& l : m->layers)
    if (!l.uploaded) return false;
  return true;
}

// The decode GEMVs read fragment-tiled copies of the weights. They cost one
// more copy of the matrices in HBM (13.5 GB for the 7B shape) and are only
// allocated once a decode path runs; an upload marks them stale and the next
// decode call re-tiles on the stream, ahead of its own launches.
int ensure_decode_weights(hb_model* m) {
  const hb_model_config& c = m->cfg;
  const size_t d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden, V = c.vocab;
  if (!m->dbase) {
    const size_t per_layer = align256((q + 2 * kv) * d * 2) + align256(d * q * 2) +
                             align256(2 * h * d * 2) + align256(d * h * 2);
    const size_t total = per_layer * c.nlayers + align256(V * d * 2);
    HIP_TRY(hipStreamSynchronize(m->ctx->stream()));
    char* base = nullptr;
    hipError_t e = hipMalloc(&base, total);
    if (e != hipSuccess)
      return fail(e == hipErrorOutOfMemory ? HB_E_OOM : HB_E_DEVICE,
                  "decode weight copy of %zu bytes: %s", total, hipGetErrorString(e));
    m->dbase = base;
    m->dbytes = total;
    size_t off = 0;
    for (auto& L : m->layers) {
      L.t_wqkv = (f16*)(base + off); off += align256((q + 2 * kv) * d * 2);
      L.t_wo = (f16*)(base + off); off += align256(d * q * 2);
      L.t_w13 = (f16*)(base + off); off += align256(2 * h * d * 2);
      L.t_w2 = (f16*)(base + off); off += align256(d * h * 2);
    }
    m->t_embed = (f16*)(base + off);
    m->dec_stale = true;
    m->wt_stale = true;
    m->graph_epoch++;
  }
  if (m->dec_stale) {
    hipStream_t st = m->ctx->stream();
    for (auto& L : m->layers) {
      HIP_TRY(tile_decode(L.wqkv, L.t_wqkv, (int)(q + 2 * kv), (int)d, st));
      HIP_TRY(tile_decode(L.wo, L.t_wo, (int)d, (int)q, st));
      HIP_TRY(tile_decode(L.w13, L.t_w13, (int)(2 * h), (int)d, st));
      HIP_TRY(tile_decode(L.w2, L.t_w2, (int)d, (int)h, st));
    }
    HIP_TRY(tile_decode(m->embed, m->t_embed, (int)V, (int)d, st));
    m->dec_stale = false;
  }
  return HB_OK;
}

// One transformer layer over T = B*S token rows (layer.rs:684-806 order).
// x -> x (in place through x2). K/V targets are either the workspace scratch
// (forward) or the KV cache (prefill for decode).
struct KVTarget {
  f16* k;
  size_t k_bstride, k_hstride;
  f16* v;  // nullable
  size_t v_bstride, v_hstride;
  // low parts for split-operand layers, same strides (v_lo nullable)
  f16 *k_lo = nullptr, *v_lo = nullptr;
};

int zero_vt_pad(hb_model* m, f16* vt, int B, int S, hipStream_t st);

// xn_ready: w.xn already holds RMSNorm1(x) (the previous layer's W2 produced
// it). next_gamma != NULL: also leave RMSNorm(x_out, next_gamma) in w.xn for
// the next layer (or the final norm); the norm is fused into the W2 split-K
// reduction when that projection splits.
// Layers l < np run on two-term fp16 operands (common.hpp): split rows for
// xn, attn, x2n and gate (GEMM K doubled, weights read once per half), Q, K,
// V with low parts, split attention; the norm that feeds layer l is written
// split when l < np. kv.k_lo / kv.v_lo must be set for those layers.
// Stage boundaries of a timed forward (hb_forward_timed): an event is
// recorded on the stream after each stage's launches, and the time between
// consecutive events is added to that stage. Null in every other forward.
enum Stage {
  ST_EMBED, ST_NORM1, ST_QKV, ST_ATTN, ST_WO, ST_WO_NORM, ST_FFN_UP, ST_FFN_DOWN, ST_FFN_NORM,
  ST_LOGITS, ST_CE, ST_COUNT
};
struct StageTimer {
  hipStream_t st;
  std::vector<hipEvent_t> ev;
  std::vector<std::pair<int, int>> tag;  // (stage, layer) that ends at ev[i]
  int layer = -1;
  hipEvent_t next(int stage) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    ev.push_back(e);
    tag.emplace_back(stage, layer);
    return e;
  }
  hipError_t mark(int stage) {
    hipEvent_t e = next(stage);
    return e ? hipEventRecord(e, st) : hipErrorOutOfMemory;
  }
  ~StageTimer() {
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  }
};
#define HB_MARK(tm, stage) \
  do {                     \
    if (tm) HIP_TRY((tm)->mark(stage)); \
  } while (0)

int run_layer(hb_model* m, int l, int B, int S, const KVTarget& kv, float* qkv_tap, bool xn_ready,
              const float* next_gamma, int np, StageTimer* tm = nullptr) {
  const hb_model_config& c = m->cfg;
  Workspace& w = m->ws;
  const LayerW& L = m->layers[l];
  hipStream_t st = m->ctx->stream();
  const int T = B * S, Sp = S_pad_of(S);
  const float alpha = alpha_of(c);
  // the norm after the last layer feeds the logits: split when every layer is
  const bool sp = l < np, sp_next = l + 1 < np || (l + 1 == c.nlayers && np == c.nlayers);
  if ((sp && (!w.split || !kv.k_lo)) || (sp_next && !w.split))
    return fail(HB_E_STATE, "split-operand buffers missing");
  const int f = sp ? 2 : 1;  // K multiplier of this layer's products

  if (tm) tm->layer = l;
  if (!xn_ready) {
    HIP_TRY(rmsnorm(w.x, c.dim, L.g1, T, c.dim, c.norm_eps, w.xn, nullptr, st, sp));
    HB_MARK(tm, ST_NORM1);
  }
  EpiQKV e{};
  e.q_dim = c.q_dim;
  e.kv_dim = c.kv_dim;
  e.hd = c.hd;
  e.S = S;
  e.heads = c.heads;
  e.kv_heads = c.kv_heads;
  e.rope = m->rope;
  e.rope_ld = m->rope_len;
  e.d_pos = nullptr;
  e.q = w.q;
  e.q_rows = Sp;
  e.k = kv.k;
  e.k_bstride = kv.k_bstride;
  e.k_hstride = kv.k_hstride;
  e.v = kv.v;
  e.v_bstride = kv.v_bstride;
  e.v_hstride = kv.v_hstride;
  e.vt = w.vt;
  e.vt_ld = Sp;
  e.tap = qkv_tap;
  if (sp) {
    e.q_lo = w.q_lo;
    e.k_lo = kv.k_lo;
    e.v_lo = kv.v_lo;
    e.vt_lo = w.vt_lo;
  }
  HIP_TRY(gemm_qkv(L.wqkv, w.xn, c.q_dim + 2 * c.kv_dim, T, f * c.dim, e, st, c.dim));
  TRY(zero_vt_pad(m, w.vt, B, S, st));
  if (sp) TRY(zero_vt_pad(m, w.vt_lo, B, S, st));
  HB_MARK(tm, ST_QKV);
  AttnPrefill a{};
  a.q = w.q;
  a.q_rows = Sp;
  a.k = kv.k;
  a.k_bstride = kv.k_bstride;
  a.k_hstride = kv.k_hstride;
  a.vt = w.vt;
  a.vt_ld = Sp;
  a.out = w.attn;
  a.B = B;
  a.S = S;
  a.H = c.heads;
  a.KVH = c.kv_heads;
  a.hd = c.hd;
  a.scale = 1.0f / sqrtf((float)c.hd);
  if (sp) {
    a.q_lo = w.q_lo;
    a.k_lo = kv.k_lo;
    a.vt_lo = w.vt_lo;
  }
  HIP_TRY(attention_prefill(a, st));
  HB_MARK(tm, ST_ATTN);
  GemmScratch so, s2;
  TRY(residual_scratch(m, c.dim, T, f * c.q_dim, so));
  HIP_TRY(gemm_residual_norm(L.wo, w.attn, c.dim, T, f * c.q_dim, EpiResidual{w.x, w.x2, c.dim, alpha},
                             NormOut{L.g2, c.norm_eps, w.xn, sp}, &so, st, c.q_dim,
                             tm ? tm->next(ST_WO) : nullptr));
  HB_MARK(tm, ST_WO_NORM);
  HIP_TRY(gemm_swiglu(L.w13, w.xn, 2 * c.hidden, T, f * c.dim, EpiSwiGLU{w.gate, nullptr, c.hidden, sp}, st,
                      c.dim));
  HB_MARK(tm, ST_FFN_UP);
  TRY(residual_scratch(m, c.dim, T, f * c.hidden, s2));
  const EpiResidual e2{w.x2, w.x, c.dim, alpha};
  if (next_gamma) {
    HIP_TRY(gemm_residual_norm(L.w2, w.gate, c.dim, T, f * c.hidden, e2,
                               NormOut{next_gamma, c.norm_eps, w.xn, sp_next}, &s2, st, c.hidden,
                               tm ? tm->next(ST_FFN_DOWN) : nullptr));
    HB_MARK(tm, ST_FFN_NORM);
  } else {
    HIP_TRY(gemm_residual(L.w2, w.gate, c.dim, T, f * c.hidden, e2, &s2, st, c.hidden));
    HB_MARK(tm, ST_FFN_DOWN);
  }
  return HB_OK;
}

KVTarget scratch_kv(hb_model* m, int B, int S) {
  const hb_model_config& c = m->cfg;
  const int Sp = S_pad_of(S);
  KVTarget t{};
  t.k = m->ws.k;
  t.k_hstride = (size_t)Sp * c.hd;
  t.k_bstride = (size_t)c.kv_heads * t.k_hstride;
  t.v = nullptr;
  t.k_lo = m->ws.k_lo;
  (void)B;
  return t;
}

}  // namespace

// Zero the V^T columns [S, S_pad) so masked (p = 0) keys never meet a NaN.
__global__ void zero_vt_pad_kernel(f16* vt, int rows, int ld, int S) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 5);
  const int c = S + (threadIdx.x & 31);
  if (r < rows && c < ld) vt[(size_t)r * ld + c] = (f16)0.f;
}

namespace {
int zero_vt_pad(hb_model* m, f16* vt, int B, int S, hipStream_t st) {
  const int Sp = S_pad_of(S);
  if (Sp == S) return HB_OK;
  const int rows = B * m->cfg.kv_heads * m->cfg.hd;
  hipLaunchKernelGGL(zero_vt_pad_kernel, dim3((rows + 3) / 4), dim3(128), 0, st, vt, rows, Sp, S);
  HIP_TRY(hipGetLastError());
  return HB_OK;
}
}  // namespace

// ---------------------------------------------------------------------------
// library / context
// ---------------------------------------------------------------------------
extern "C" const char* hb_backend_name(void) { return "hip-gfx950"; }
extern "C" const char* hb_last_error(void) { return g_err.c_str(); }

extern "C" int hb_debug_inject_error(int code) {
  g_inject.store(code);
  return HB_OK;
}

extern "C" int hb_device_count(int* out) {
  HB_INJECT_CHECK();
  if (!out) return fail(HB_E_INVALID, "null out");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *out = n;
  return HB_OK;
}

// ---- scratch of the allocation-free entry point (hb_op_wo_fwd_noalloc) ----
// The split-K partial sums of hb_op_wo_fwd_noalloc live in this file-scope
// device array -- one copy on every GPU the library runs on, held until the
// process ends -- instead of memory the library allocates. 16 MiB suffices
// for every shape: gemm_splits aims the split count S at 256 workgroups of
// 128x128 tiles (S <= 256 / tiles), so S * T * N <= 256 * 128 * 128 floats.
constexpr size_t NOALLOC_SCRATCH_FLOATS = (size_t)256 * 128 * 128;
static __device__ __align__(256) float scratch[NOALLOC_SCRATCH_FLOATS];

// Device address of `scratch` on each device, looked up once per device (with
// that device current) when the first context on it is created. Host code
// uses these addresses, never the array's name (a host-side stand-in).
constexpr int NOALLOC_MAX_DEVICES = 64;
static float* g_scratch_dev[NOALLOC_MAX_DEVICES];
// Last use of each device's array: calls outside a graph capture wait for it
// on their own stream and record it afterwards, so two calls from different
// streams (contexts, hb_ctx_set_stream) run one after the other instead of
// sharing the partial sums.
static hipEvent_t g_scratch_ev[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

static int scratch_setup(int device) {
  if (device < 0 || device >= NOALLOC_MAX_DEVICES) return fail(HB_E_DEVICE, "device %d beyond the scratch table", device);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[device]) return HB_OK;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) return fail(HB_E_DEVICE, "scratch address on device %d: %s", device, hipGetErrorString(e));
  if (!g_scratch_ev[device]) e = hipEventCreateWithFlags(&g_scratch_ev[device], hipEventDisableTiming);
  if (e != hipSuccess) return fail(HB_E_DEVICE, "scratch event on device %d: %s", device, hipGetErrorString(e));
  g_scratch_dev[device] = (float*)p;
  return HB_OK;
}

static float* scratch_of(int device) {
  if (device < 0 || device >= NOALLOC_MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return g_scratch_dev[device];
}

extern "C" int hb_ctx_create(int device, hb_ctx** out) {
  HB_INJECT_CHECK();
  if (!out) return fail(HB_E_INVALID, "null out");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return fail(HB_E_DEVICE, "no HIP device");
  if (device < 0 || device >= n) return fail(HB_E_INVALID, "device %d out of range [0,%d)", device, n);
  DeviceGuard g(device);
  hb_ctx* c = new hb_ctx();
  c->device = device;
  // The context's own stream is a blocking stream: it orders with work that
  // callers put on the null stream (torch's default). Graph capture uses a
  // separate non-blocking stream.
  hipError_t e = hipStreamCreateWithFlags(&c->own, hipStreamDefault);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->capture, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&c->d_err, 256);
  if (e == hipSuccess) e = hipMemset(c->d_err, 0, 256);
  if (e != hipSuccess) {
    if (c->own) (void)hipStreamDestroy(c->own);
    if (c->capture) (void)hipStreamDestroy(c->capture);
    delete c;
    return fail(HB_E_DEVICE, "context setup failed: %s", hipGetErrorString(e));
  }
  const int r = scratch_setup(device);
  if (r != HB_OK) {
    (void)hipFree(c->d_err);
    (void)hipStreamDestroy(c->own);
    (void)hipStreamDestroy(c->capture);
    delete c;
    return r;
  }
  *out = c;
  return HB_OK;
}

extern "C" int hb_ctx_destroy(hb_ctx* c) {
  if (!c) return HB_OK;
  DeviceGuard g(c->device);
  (void)hipDeviceSynchronize();  // the caller's stream may already be gone
  (void)hipFree(c->d_err);
  (void)hipStreamDestroy(c->own);
  (void)hipStreamDestroy(c->capture);
  delete c;
  return HB_OK;
}

extern "C" int hb_ctx_set_stream(hb_ctx* c, void* s) {
  HB_INJECT_CHECK();
  if (!c) return fail(HB_E_INVALID, "null ctx");
  c->user = (hipStream_t)s;
  return HB_OK;
}

extern "C" int hb_ctx_get_stream(hb_ctx* c, void** s) {
  HB_INJECT_CHECK();
  if (!c || !s) return fail(HB_E_INVALID, "null argument");
  *s = (void*)c->stream();
  return HB_OK;
}

extern "C" int hb_ctx_synchronize(hb_ctx* c) {
  HB_INJECT_CHECK();
  if (!c) return fail(HB_E_INVALID, "null ctx");
  DeviceGuard g(c->device);
  HIP_TRY(hipStreamSynchronize(c->stream()));
  return check_err_word(c);
}

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
extern "C" int hb_config_validate(hb_model_config* c) {
  HB_INJECT_CHECK();
  if (!c) return fail(HB_E_INVALID, "null config");
  if (c->rope_theta == 0.f) c->rope_theta = 10000.0f;
  if (c->norm_eps == 0.f) c->norm_eps = 1e-5f;
  if (c->residual_alpha == 0.f && c->nlayers > 0)
    c->residual_alpha = 1.0f / sqrtf(2.0f * (float)c->nlayers);
  if (!(c->softcap >= 0.f)) return fail(HB_E_CONFIG, "softcap must be >= 0");
  return validate_config(*c);
}

extern "C" int hb_model_create(hb_ctx* ctx, const hb_model_config* cfg_in, int dtype,
                               hb_model** out) {
  HB_INJECT_CHECK();
  if (!ctx || !cfg_in || !out) return fail(HB_E_INVALID, "null argument");
  *out = nullptr;
  if (dtype != HB_DTYPE_F16) return fail(HB_E_CONFIG, "unsupported dtype %d", dtype);
  hb_model_config c = *cfg_in;
  TRY(hb_config_validate(&c));
  DeviceGuard g(ctx->device);

  const size_t d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden, V = c.vocab;
  const size_t per_layer = align256((q + 2 * kv) * d * 2) + align256(d * q * 2) +
                           align256(2 * h * d * 2) + align256(d * h * 2) + 2 * align256(d * 4);
  const size_t total = per_layer * c.nlayers + align256(V * d * 2) + align256(d * 4);
  char* base = nullptr;
  hipError_t e = hipMalloc(&base, total);
  if (e != hipSuccess)
    return fail(e == hipErrorOutOfMemory ? HB_E_OOM : HB_E_DEVICE,
                "weight allocation of %zu bytes failed: %s", total, hipGetErrorString(e));
  hb_model* m = new hb_model();
  m->ctx = ctx;
  m->device = ctx->device;
  m->cfg = c;
  m->wbase = base;
  m->wbytes = total;
  m->layers.resize(c.nlayers);
  size_t off = 0;
  for (int l = 0; l < c.nlayers; ++l) {
    LayerW& L = m->layers[l];
    L.wqkv = (f16*)(base + off); off += align256((q + 2 * kv) * d * 2);
    L.wo = (f16*)(base + off); off += align256(d * q * 2);
    L.w13 = (f16*)(base + off); off += align256(2 * h * d * 2);
    L.w2 = (f16*)(base + off); off += align256(d * h * 2);
    L.g1 = (float*)(base + off); off += align256(d * 4);
    L.g2 = (float*)(base + off); off += align256(d * 4);
  }
  m->embed = (f16*)(base + off); off += align256(V * d * 2);
  m->gamma_f = (float*)(base + off);
  int r = ensure_rope(m, c.seq);
  if (r != HB_OK) {
    (void)hipFree(base);
    delete m;
    return r;
  }
  *out = m;
  return HB_OK;
}

// Destroy functions touch only their own object: callers (for instance a
// garbage collector finalising a reference cycle) may destroy a context or
// model before the objects created from it.
extern "C" int hb_model_destroy(hb_model* m) {
  if (!m) return HB_OK;
  DeviceGuard g(m->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(m->wbase);
  if (m->dbase) (void)hipFree(m->dbase);
  if (m->splitk) (void)hipFree(m->splitk);
  if (m->rope) (void)hipFree(m->rope);
  if (m->staging) (void)hipFree(m->staging);
  if (m->ws.base) (void)hipFree(m->ws.base);
  if (m->fwd_exec) (void)hipGraphExecDestroy(m->fwd_exec);
  if (m->fwd_graph) (void)hipGraphDestroy(m->fwd_graph);
  train_free(m->train);
  delete m;
  return HB_OK;
}

extern "C" int hb_model_get_config(const hb_model* m, hb_model_config* out) {
  HB_INJECT_CHECK();
  if (!m || !out) return fail(HB_E_INVALID, "null argument");
  *out = m->cfg;
  return HB_OK;
}

extern "C" int hb_model_weight_bytes(const hb_model* m, uint64_t* out) {
  HB_INJECT_CHECK();
  if (!m || !out) return fail(HB_E_INVALID, "null argument");
  *out = m->wbytes;
  return HB_OK;
}

extern "C" int hb_model_set_precise_layers(hb_model* m, int n) {
  HB_INJECT_CHECK();
  if (!m) return fail(HB_E_INVALID, "null model");
  if (n < 0 || n > m->cfg.nlayers) return fail(HB_E_INVALID, "precise layers %d outside [0, %d]", n, m->cfg.nlayers);
  m->precise_layers = n;
  return HB_OK;
}

extern "C" int hb_model_get_precise_layers(const hb_model* m, int* out) {
  HB_INJECT_CHECK();
  if (!m || !out) return fail(HB_E_INVALID, "null argument");
  *out = m->precise_layers;
  return HB_OK;
}

extern "C" int hb_model_set_softcap(hb_model* m, float softcap) {
  HB_INJECT_CHECK();
  if (!m) return fail(HB_E_INVALID, "null model");
  if (!(softcap >= 0.f)) return fail(HB_E_INVALID, "softcap must be >= 0");
  if (softcap != m->cfg.softcap) {
    m->cfg.softcap = softcap;
    // The decode graphs bake the softcap into their logits launch.
    m->graph_epoch++;
  }
  return HB_OK;
}

namespace {
// Host fp32 [R][C] -> staging -> packed fp16.
int upload_packed(hb_model* m, const float* src, int R, int C, f16* dst, int ld, int row0, int mode) {
  TRY(ensure_staging(m, (size_t)R * C));
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(m->staging, src, (size_t)R * C * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(repack(m->staging, R, C, dst, ld, row0, mode, st));
  HIP_TRY(hipStreamSynchronize(st));
  return HB_OK;
}
int upload_f32(hb_model* m, const float* src, size_t n, float* dst) {
  HIP_TRY(hipMemcpyAsync(dst, src, n * 4, hipMemcpyHostToDevice, m->ctx->stream()));
  HIP_TRY(hipStreamSynchronize(m->ctx->stream()));
  return HB_OK;
}
}  // namespace

extern "C" int hb_model_upload_layer(hb_model* m, int layer, const float* wq, const float* wk,
                                     const float* wv, const float* wo, const float* w1,
                                     const float* w3, const float* w2, const float* g1,
                                     const float* g2) {
  HB_INJECT_CHECK();
  if (!m) return fail(HB_E_INVALID, "null model");
  if (layer < 0 || layer >= m->cfg.nlayers) return fail(HB_E_INVALID, "layer %d out of range", layer);
  if (!wq || !wk || !wv || !wo || !w1 || !w3 || !w2 || !g1 || !g2)
    return fail(HB_E_INVALID, "null weight pointer");
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  LayerW& L = m->layers[layer];
  const int d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden;
  TRY(upload_packed(m, wq, d, q, L.wqkv, d, 0, 0));
  TRY(upload_packed(m, wk, d, kv, L.wqkv, d, q, 0));
  TRY(upload_packed(m, wv, d, kv, L.wqkv, d, q + kv, 0));
  TRY(upload_packed(m, wo, q, d, L.wo, q, 0, 0));
  TRY(upload_packed(m, w1, d, h, L.w13, d, 0, 1));
  TRY(upload_packed(m, w3, d, h, L.w13, d, 2, 1));
  TRY(upload_packed(m, w2, d, h, L.w2, h, 0, 2));
  TRY(upload_f32(m, g1, d, L.g1));
  TRY(upload_f32(m, g2, d, L.g2));
  L.uploaded = true;
  m->dec_stale = true;
  m->wt_stale = true;
  return HB_OK;
}

extern "C" int hb_model_upload_embed(hb_model* m, const float* embed, const float* gamma_final) {
  HB_INJECT_CHECK();
  if (!m || !embed || !gamma_final) return fail(HB_E_INVALID, "null argument");
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  // Upload in row chunks to bound the staging buffer.
  const int rows_per = std::max(1, (int)std::min<size_t>(c.vocab, (64u << 20) / c.dim));
  for (int r0 = 0; r0 < c.vocab; r0 += rows_per) {
    const int rows = std::min(rows_per, c.vocab - r0);
    TRY(upload_packed(m, embed + (size_t)r0 * c.dim, rows, c.dim, m->embed, c.dim, r0, 2));
  }
  TRY(upload_f32(m, gamma_final, c.dim, m->gamma_f));
  m->embed_uploaded = true;
  m->dec_stale = true;
  m->wt_stale = true;
  return HB_OK;
}

extern "C" int hb_model_init_synthetic(hb_model* m, uint64_t seed, float std) {
  HB_INJECT_CHECK();
  if (!m) return fail(HB_E_INVALID, "null model");
  if (!(std > 0.f)) return fail(HB_E_INVALID, "std must be positive");
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  hipStream_t st = m->ctx->stream();
  const float sc = hb_normal_scale(std);
  const int d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden;
  // Same staging -> repack path as a host upload, with the fp32 source array
  // generated on the device instead of copied from the host.
  auto put = [&](uint64_t id, int R, int C, f16* dst, int ld, int row0, int mode) -> int {
    TRY(ensure_staging(m, (size_t)R * C));
    HIP_TRY(synth_f32(seed, id, sc, 0, (size_t)R * C, m->staging, st));
    HIP_TRY(repack(m->staging, R, C, dst, ld, row0, mode, st));
    return HB_OK;
  };
  for (int l = 0; l < c.nlayers; ++l) {
    LayerW& L = m->layers[l];
    const uint64_t id = 16ull * l;
    TRY(put(id + 0, d, q, L.wqkv, d, 0, 0));
    TRY(put(id + 1, d, kv, L.wqkv, d, q, 0));
    TRY(put(id + 2, d, kv, L.wqkv, d, q + kv, 0));
    TRY(put(id + 3, q, d, L.wo, q, 0, 0));
    TRY(put(id + 4, d, h, L.w13, d, 0, 1));
    TRY(put(id + 5, d, h, L.w13, d, 2, 1));
    TRY(put(id + 6, d, h, L.w2, h, 0, 2));
    HIP_TRY(fill_f32(L.g1, 1.0f, d, st));
    HIP_TRY(fill_f32(L.g2, 1.0f, d, st));
    L.uploaded = true;
  }
  const int rows_per = std::max(1, (int)std::min<size_t>(c.vocab, (64u << 20) / c.dim));
  for (int r0 = 0; r0 < c.vocab; r0 += rows_per) {
    const int rows = std::min(rows_per, c.vocab - r0);
    TRY(ensure_staging(m, (size_t)rows * d));
    HIP_TRY(synth_f32(seed, HB_SYNTH_EMBED_ID, sc, (uint64_t)r0 * d, (size_t)rows * d, m->staging, st));
    HIP_TRY(repack(m->staging, rows, d, m->embed, d, r0, 2, st));
  }
  HIP_TRY(fill_f32(m->gamma_f, 1.0f, d, st));
  HIP_TRY(hipStreamSynchronize(st));
  m->embed_uploaded = true;
  m->dec_stale = true;
  m->wt_stale = true;
  return HB_OK;
}

// ---------------------------------------------------------------------------
// optimizer
// ---------------------------------------------------------------------------
namespace {
enum { OPT_MATRIX = 0, OPT_EMBED = 1, OPT_GAMMA = 2 };
// A run of elements that one AdamW launch updates: arena offset, length,
// learning-rate group and the model tensor (fp16 weights or fp32 gammas)
// rewritten from the new master values.
struct OptSeg {
  size_t off, n;
  int group;
  f16* d16;
  float* d32;
};
struct OptLayerOff {
  size_t wqkv, wo, w13, w2, g1, g2;
};

// f32::powi as the reference's bias corrections evaluate it (cpu/adam.rs:113-114):
// exponentiation by squaring in fp32 (the compiler-rt __powisf2 algorithm
// that llvm.powi.f32 lowers to).
float powi_f32(float a, int b) {
  const bool recip = b < 0;
  float r = 1.0f;
  for (;;) {
    if (b & 1) r *= a;
    b /= 2;
    if (b == 0) break;
    a *= a;
  }
  return recip ? 1.0f / r : r;
}

float learning_rate_f32(const hb_train_config& tc, uint32_t step) {
  if (step < tc.warmup_steps) return tc.max_lr * (float)(step + 1) / (float)tc.warmup_steps;
  const float decay = (float)(step - tc.warmup_steps) / (float)(tc.total_steps - tc.warmup_steps);
  const float min_lr = tc.max_lr * tc.min_lr_frac;
  const float pi = 3.14159265358979323846f;
  return min_lr + 0.5f * (1.0f + cosf(pi * decay)) * (tc.max_lr - min_lr);
}

// out[i*C + j] = packed element that repack(mode, row0, ld) wrote for src[i][j].
void unpack_host(const float* packed, int R, int C, int ld, int row0, int mode, float* out) {
  for (int i = 0; i < R; ++i)
    for (int j = 0; j < C; ++j) {
      const int row = mode == 0 ? row0 + j : mode == 1 ? ((j >> 1) << 2) + (j & 1) + row0 : row0 + i;
      out[(size_t)i * C + j] = packed[(size_t)row * ld + (mode == 2 ? j : i)];
    }
}

int validate_train_config(const hb_train_config& tc) {
  if (!(tc.beta1 >= 0.f && tc.beta1 < 1.f && tc.beta2 >= 0.f && tc.beta2 < 1.f))
    return fail(HB_E_INVALID, "betas must be in [0, 1)");
  if (!(tc.eps > 0.f) || !(tc.loss_scale > 0.f) || tc.accum_steps == 0 || !(tc.grad_clip > 0.f))
    return fail(HB_E_INVALID, "eps, loss_scale, accum_steps and grad_clip must be positive");
  if (tc.warmup_steps == 0 || tc.total_steps <= tc.warmup_steps)
    return fail(HB_E_INVALID, "need 0 < warmup_steps < total_steps");
  return HB_OK;
}
}  // namespace

struct hb_opt {
  hb_model* model = nullptr;
  int device = 0;
  hb_train_config tc{};
  void* base = nullptr;
  size_t n = 0;  // floats per arena
  float *p = nullptr, *g = nullptr, *m = nullptr, *v = nullptr;
  std::vector<OptSeg> segs;
  std::vector<OptLayerOff> lo;
  size_t embed_off = 0, gf_off = 0;
  double* partials = nullptr;
  float* scal = nullptr;  // [0] norm, [1] train_step scale, [2] clip_grads factor
  // The gradient arena holds zeros (creation, hb_opt_zero_grads) and nothing
  // has written it since: the next training backward stores instead of adding.
  // Never set again once hb_opt_grad_arena has handed out the raw pointer
  // (the caller may write through it at any time).
  bool grads_zero = true;
  bool arena_exposed = false;
  // hb_opt_zero_grads left the clearing to the first consumer: the arena is
  // logically zero but its memory is stale until opt_materialize (or a
  // training backward, which stores every element) runs.
  bool lazy_zero = false;
  // Sums of squares taken while a training backward wrote the gradients (one
  // fp32 per output tile or gamma block, then the embedding's fp64 partials):
  // valid (sq_ready) until anything else writes the arena; the norm then
  // needs no second pass over it.
  float* sq_slots = nullptr;
  long sq_cap = 0, sq_n = 0;
  double* sq_embed = nullptr;  // [SUMSQ_BLOCKS]
  bool sq_ready = false;
};

extern "C" int hb_learning_rate(const hb_train_config* tc, uint32_t step, float* out) {
  HB_INJECT_CHECK();
  if (!tc || !out) return fail(HB_E_INVALID, "null argument");
  TRY(validate_train_config(*tc));
  *out = learning_rate_f32(*tc, step);
  return HB_OK;
}

extern "C" int hb_opt_create(hb_model* mo, const hb_train_config* tc, hb_opt** out) {
  HB_INJECT_CHECK();
  if (!mo || !tc || !out) return fail(HB_E_INVALID, "null argument");
  *out = nullptr;
  TRY(validate_train_config(*tc));
  DeviceGuard gd(mo->ctx->device);
  const hb_model_config& c = mo->cfg;
  const size_t d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden, V = c.vocab;
  hb_opt* o = new hb_opt();
  o->model = mo;
  o->device = mo->device;
  o->tc = *tc;
  size_t off = 0;
  std::vector<OptSeg> raw;
  for (int l = 0; l < c.nlayers; ++l) {
    LayerW& L = mo->layers[l];
    OptLayerOff lo{};
    auto add = [&](size_t n, int group, f16* d16, float* d32) {
      raw.push_back(OptSeg{off, n, group, d16, d32});
      const size_t at = off;
      off += n;
      return at;
    };
    lo.wqkv = add((q + 2 * kv) * d, OPT_MATRIX, L.wqkv, nullptr);
    lo.wo = add(d * q, OPT_MATRIX, L.wo, nullptr);
    lo.w13 = add(2 * h * d, OPT_MATRIX, L.w13, nullptr);
    lo.w2 = add(d * h, OPT_MATRIX, L.w2, nullptr);
    lo.g1 = add(d, OPT_GAMMA, nullptr, L.g1);
    lo.g2 = add(d, OPT_GAMMA, nullptr, L.g2);
    o->lo.push_back(lo);
  }
  o->embed_off = off;
  raw.push_back(OptSeg{off, V * d, OPT_EMBED, mo->embed, nullptr});
  off += V * d;
  o->gf_off = off;
  raw.push_back(OptSeg{off, d, OPT_GAMMA, nullptr, mo->gamma_f});
  off += d;
  o->n = off;
  // one launch per run of same-group tensors that are contiguous in both the
  // arenas and the model's weights (a layer's four matrices are)
  for (const OptSeg& sg : raw) {
    if (!o->segs.empty()) {
      OptSeg& b = o->segs.back();
      const bool same = b.group == sg.group && b.off + b.n == sg.off &&
                        ((b.d16 && sg.d16 && b.d16 + b.n == sg.d16) ||
                         (b.d32 && sg.d32 && b.d32 + b.n == sg.d32));
      if (same) {
        b.n += sg.n;
        continue;
      }
    }
    o->segs.push_back(sg);
  }
  const size_t arena = align256(o->n * 4);
  const size_t total = 4 * arena + align256(SUMSQ_BLOCKS * 8) + 256;
  char* b = nullptr;
  hipError_t e = hipMalloc(&b, total);
  if (e != hipSuccess) {
    delete o;
    return fail(e == hipErrorOutOfMemory ? HB_E_OOM : HB_E_DEVICE,
                "optimizer state of %zu bytes: %s", total, hipGetErrorString(e));
  }
  o->base = b;
  o->p = (float*)b;
  o->g = (float*)(b + arena);
  o->m = (float*)(b + 2 * arena);
  o->v = (float*)(b + 3 * arena);
  o->partials = (double*)(b + 4 * arena);
  o->scal = (float*)(b + 4 * arena + align256(SUMSQ_BLOCKS * 8));
  hipStream_t st = mo->ctx->stream();
  auto init = [&]() -> int {
    HIP_TRY(hipMemsetAsync(b + arena, 0, 3 * arena, st));  // g, m, v
    for (const OptSeg& sg : raw) {
      if (sg.d16)
        HIP_TRY(widen_f16(sg.d16, o->p + sg.off, sg.n, st));
      else
        HIP_TRY(hipMemcpyAsync(o->p + sg.off, sg.d32, sg.n * 4, hipMemcpyDeviceToDevice, st));
    }
    HIP_TRY(hipStreamSynchronize(st));
    return HB_OK;
  };
  int r = init();
  if (r != HB_OK) {
    (void)hipFree(b);
    delete o;
    return r;
  }
  *out = o;
  return HB_OK;
}

extern "C" int hb_opt_destroy(hb_opt* o) {
  if (!o) return HB_OK;
  DeviceGuard g(o->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(o->base);
  if (o->sq_slots) (void)hipFree(o->sq_slots);
  if (o->sq_embed) (void)hipFree(o->sq_embed);
  delete o;
  return HB_OK;
}

namespace {
// Host fp32 [R][C] (reference layout) -> staging -> packed fp32 at dst32 and,
// when dst16 is set, packed fp16 at dst16.
int opt_put(hb_model* m, const float* src, int R, int C, float* dst32, f16* dst16, int ld, int row0,
            int mode) {
  TRY(ensure_staging(m, (size_t)R * C));
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(m->staging, src, (size_t)R * C * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(repack_f32(m->staging, R, C, dst32, ld, row0, mode, st));
  if (dst16) HIP_TRY(repack(m->staging, R, C, dst16, ld, row0, mode, st));
  HIP_TRY(hipStreamSynchronize(st));
  return HB_OK;
}

// Reference-layout layer tensors into arena `a` (and the model when `model`).
int opt_put_layer(hb_opt* o, float* a, bool model, int layer, const float* const w[9]) {
  hb_model* m = o->model;
  const hb_model_config& c = m->cfg;
  LayerW& L = m->layers[layer];
  const OptLayerOff& lo = o->lo[layer];
  const int d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden;
  TRY(opt_put(m, w[0], d, q, a + lo.wqkv, model ? L.wqkv : nullptr, d, 0, 0));
  TRY(opt_put(m, w[1], d, kv, a + lo.wqkv, model ? L.wqkv : nullptr, d, q, 0));
  TRY(opt_put(m, w[2], d, kv, a + lo.wqkv, model ? L.wqkv : nullptr, d, q + kv, 0));
  TRY(opt_put(m, w[3], q, d, a + lo.wo, model ? L.wo : nullptr, q, 0, 0));
  TRY(opt_put(m, w[4], d, h, a + lo.w13, model ? L.w13 : nullptr, d, 0, 1));
  TRY(opt_put(m, w[5], d, h, a + lo.w13, model ? L.w13 : nullptr, d, 2, 1));
  TRY(opt_put(m, w[6], d, h, a + lo.w2, model ? L.w2 : nullptr, h, 0, 2));
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(a + lo.g1, w[7], d * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(a + lo.g2, w[8], d * 4, hipMemcpyHostToDevice, st));
  if (model) {
    HIP_TRY(hipMemcpyAsync(L.g1, w[7], d * 4, hipMemcpyHostToDevice, st));
    HIP_TRY(hipMemcpyAsync(L.g2, w[8], d * 4, hipMemcpyHostToDevice, st));
    L.uploaded = true;
    m->dec_stale = true;
    m->wt_stale = true;
  }
  HIP_TRY(hipStreamSynchronize(st));
  return HB_OK;
}

int opt_put_embed(hb_opt* o, float* a, bool model, const float* embed, const float* gf) {
  hb_model* m = o->model;
  const hb_model_config& c = m->cfg;
  const int rows_per = std::max(1, (int)std::min<size_t>(c.vocab, (64u << 20) / c.dim));
  for (int r0 = 0; r0 < c.vocab; r0 += rows_per) {
    const int rows = std::min(rows_per, c.vocab - r0);
    TRY(opt_put(m, embed + (size_t)r0 * c.dim, rows, c.dim, a + o->embed_off,
                model ? m->embed : nullptr, c.dim, r0, 2));
  }
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(a + o->gf_off, gf, c.dim * 4, hipMemcpyHostToDevice, st));
  if (model) {
    HIP_TRY(hipMemcpyAsync(m->gamma_f, gf, c.dim * 4, hipMemcpyHostToDevice, st));
    m->embed_uploaded = true;
    m->dec_stale = true;
    m->wt_stale = true;
  }
  HIP_TRY(hipStreamSynchronize(st));
  return HB_OK;
}

float* opt_arena(hb_opt* o, int which) {
  return which == 0 ? o->p : which == 1 ? o->m : which == 2 ? o->v : which == 3 ? o->g : nullptr;
}

// Device part of update_weights: one fused AdamW launch per segment.
int opt_update(hb_opt* o, uint32_t t, float lr, float grad_scale, const float* d_gscale) {
  const hb_train_config& tc = o->tc;
  hipStream_t st = o->model->ctx->stream();
  AdamW h{};
  h.b1 = tc.beta1;
  h.b2 = tc.beta2;
  h.omb1 = 1.0f - tc.beta1;
  h.omb2 = 1.0f - tc.beta2;
  h.eps = tc.eps;
  h.bc1 = 1.0f / (1.0f - powi_f32(tc.beta1, (int)t));
  h.bc2 = 1.0f / (1.0f - powi_f32(tc.beta2, (int)t));
  h.gscale = grad_scale;
  const float matrix_lr = lr * tc.matrix_lr_scale, embed_lr = lr * tc.embed_lr_scale;
  hb_model* mo = o->model;
  TrainState* ts = mo->train;
  const bool tiled = ts && ts->wtbase;  // keep the backward's transposed copies current
  for (const OptSeg& sg : o->segs) {
    AdamW hs = h;
    hs.lr = sg.group == OPT_MATRIX ? matrix_lr : sg.group == OPT_EMBED ? embed_lr : lr;
    hs.wd = sg.group == OPT_MATRIX ? tc.weight_decay : 0.0f;
    if (tiled && sg.group != OPT_GAMMA) continue;
    HIP_TRY(adamw(o->p + sg.off, o->g + sg.off, o->m + sg.off, o->v + sg.off, sg.d16, sg.d32, sg.n,
                  hs, d_gscale, st));
  }
  if (tiled) {
    const hb_model_config& c = mo->cfg;
    const int d = c.dim, q = c.q_dim, h2 = 2 * c.hidden, hh = c.hidden, qkv = c.q_dim + 2 * c.kv_dim;
    AdamW hm = h, he = h;
    hm.lr = matrix_lr;
    hm.wd = tc.weight_decay;
    he.lr = embed_lr;
    he.wd = 0.0f;
    auto upd = [&](size_t off, f16* dst, f16* dstT, int R, int C, int ldT, const AdamW& hp) {
      return adamw_tiled(o->p + off, o->g + off, o->m + off, o->v + off, dst, dstT, R, C, ldT, hp,
                         d_gscale, st);
    };
    for (int l = 0; l < c.nlayers; ++l) {
      const OptLayerOff& lo = o->lo[l];
      const LayerW& L = mo->layers[l];
      HIP_TRY(upd(lo.wqkv, L.wqkv, ts->wqkvT[l], qkv, d, qkv, hm));
      HIP_TRY(upd(lo.wo, L.wo, ts->woT[l], d, q, d, hm));
      HIP_TRY(upd(lo.w13, L.w13, ts->w13T[l], h2, d, h2, hm));
      HIP_TRY(upd(lo.w2, L.w2, ts->w2T[l], d, hh, d, hm));
    }
    HIP_TRY(upd(o->embed_off, mo->embed, ts->eT, c.vocab, d, (int)round64(c.vocab), he));
  }
  mo->dec_stale = true;
  mo->wt_stale = !tiled;
  return HB_OK;
}

int opt_norm(hb_opt* o, ClipCfg cc) {
  hipStream_t st = o->model->ctx->stream();
  if (o->sq_ready)
    HIP_TRY(combine_sumsq(o->sq_slots, o->sq_n, o->sq_embed, o->partials, st));
  else
    HIP_TRY(grad_sumsq(o->g, o->n, o->partials, st));
  HIP_TRY(grad_clip_scale(o->partials, cc, o->scal, st));
  return HB_OK;
}

int opt_read_norm(hb_opt* o, float* out) {
  hipStream_t st = o->model->ctx->stream();
  HIP_TRY(hipMemcpyAsync(out, o->scal, 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return HB_OK;
}
}  // namespace

// Clears a lazily zeroed gradient arena before anything but a training
// backward reads it or writes part of it.
static int opt_materialize(hb_opt* o) {
  if (!o->lazy_zero) return HB_OK;
  HIP_TRY(fill_f32(o->g, 0.0f, o->n, o->model->ctx->stream()));
  o->lazy_zero = false;
  return HB_OK;
}

#define HB_OPT_CHECK(o)                                        \
  do {                                                         \
    HB_INJECT_CHECK();                                         \
    if (!(o)) return fail(HB_E_INVALID, "null optimizer");     \
  } while (0)

extern "C" int hb_opt_upload_layer(hb_opt* o, int layer, const float* wq, const float* wk,
                                   const float* wv, const float* wo, const float* w1,
                                   const float* w3, const float* w2, const float* g1,
                                   const float* g2) {
  HB_OPT_CHECK(o);
  if (layer < 0 || layer >= o->model->cfg.nlayers) return fail(HB_E_INVALID, "layer %d out of range", layer);
  const float* w[9] = {wq, wk, wv, wo, w1, w3, w2, g1, g2};
  for (const float* x : w)
    if (!x) return fail(HB_E_INVALID, "null weight pointer");
  DeviceGuard g(o->device);
  return opt_put_layer(o, o->p, true, layer, w);
}

extern "C" int hb_opt_upload_embed(hb_opt* o, const float* embed, const float* gamma_final) {
  HB_OPT_CHECK(o);
  if (!embed || !gamma_final) return fail(HB_E_INVALID, "null argument");
  DeviceGuard g(o->device);
  return opt_put_embed(o, o->p, true, embed, gamma_final);
}

extern "C" int hb_opt_init_synthetic(hb_opt* o, uint64_t seed, float std) {
  HB_OPT_CHECK(o);
  if (!(std > 0.f)) return fail(HB_E_INVALID, "std must be positive");
  DeviceGuard gd(o->device);
  hb_model* m = o->model;
  TRY(hb_model_init_synthetic(m, seed, std));
  const hb_model_config& c = m->cfg;
  hipStream_t st = m->ctx->stream();
  const float sc = hb_normal_scale(std);
  const int d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden;
  // the same seeded fp32 arrays hb_model_init_synthetic generated, packed in fp32
  auto put = [&](uint64_t id, int R, int C, float* dst, int ld, int row0, int mode) -> int {
    TRY(ensure_staging(m, (size_t)R * C));
    HIP_TRY(synth_f32(seed, id, sc, 0, (size_t)R * C, m->staging, st));
    HIP_TRY(repack_f32(m->staging, R, C, dst, ld, row0, mode, st));
    return HB_OK;
  };
  for (int l = 0; l < c.nlayers; ++l) {
    const OptLayerOff& lo = o->lo[l];
    const uint64_t id = 16ull * l;
    TRY(put(id + 0, d, q, o->p + lo.wqkv, d, 0, 0));
    TRY(put(id + 1, d, kv, o->p + lo.wqkv, d, q, 0));
    TRY(put(id + 2, d, kv, o->p + lo.wqkv, d, q + kv, 0));
    TRY(put(id + 3, q, d, o->p + lo.wo, q, 0, 0));
    TRY(put(id + 4, d, h, o->p + lo.w13, d, 0, 1));
    TRY(put(id + 5, d, h, o->p + lo.w13, d, 2, 1));
    TRY(put(id + 6, d, h, o->p + lo.w2, h, 0, 2));
    HIP_TRY(fill_f32(o->p + lo.g1, 1.0f, d, st));
    HIP_TRY(fill_f32(o->p + lo.g2, 1.0f, d, st));
  }
  const int rows_per = std::max(1, (int)std::min<size_t>(c.vocab, (64u << 20) / c.dim));
  for (int r0 = 0; r0 < c.vocab; r0 += rows_per) {
    const int rows = std::min(rows_per, c.vocab - r0);
    TRY(ensure_staging(m, (size_t)rows * d));
    HIP_TRY(synth_f32(seed, HB_SYNTH_EMBED_ID, sc, (uint64_t)r0 * d, (size_t)rows * d, m->staging, st));
    HIP_TRY(repack_f32(m->staging, rows, d, o->p + o->embed_off, d, r0, 2, st));
  }
  HIP_TRY(fill_f32(o->p + o->gf_off, 1.0f, d, st));
  HIP_TRY(hipStreamSynchronize(st));
  return HB_OK;
}

extern "C" int hb_opt_upload_grads_layer(hb_opt* o, int layer, const float* dwq, const float* dwk,
                                         const float* dwv, const float* dwo, const float* dw1,
                                         const float* dw3, const float* dw2, const float* dg1,
                                         const float* dg2) {
  HB_OPT_CHECK(o);
  if (layer < 0 || layer >= o->model->cfg.nlayers) return fail(HB_E_INVALID, "layer %d out of range", layer);
  const float* w[9] = {dwq, dwk, dwv, dwo, dw1, dw3, dw2, dg1, dg2};
  for (const float* x : w)
    if (!x) return fail(HB_E_INVALID, "null gradient pointer");
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  o->grads_zero = false;
  o->sq_ready = false;
  return opt_put_layer(o, o->g, false, layer, w);
}

extern "C" int hb_opt_upload_grads_embed(hb_opt* o, const float* dembed, const float* dgamma_final) {
  HB_OPT_CHECK(o);
  if (!dembed || !dgamma_final) return fail(HB_E_INVALID, "null argument");
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  o->grads_zero = false;
  o->sq_ready = false;
  return opt_put_embed(o, o->g, false, dembed, dgamma_final);
}

extern "C" int hb_opt_zero_grads(hb_opt* o) {
  HB_OPT_CHECK(o);
  DeviceGuard g(o->device);
  o->sq_ready = false;
  if (o->arena_exposed) {
    // the caller may read or write the memory directly: clear it now
    HIP_TRY(fill_f32(o->g, 0.0f, o->n, o->model->ctx->stream()));
    o->grads_zero = false;
    o->lazy_zero = false;
  } else {
    o->grads_zero = true;
    o->lazy_zero = true;
  }
  return HB_OK;
}

extern "C" int hb_opt_grad_arena(hb_opt* o, float** d_grads, uint64_t* n_floats) {
  HB_OPT_CHECK(o);
  if (!d_grads || !n_floats) return fail(HB_E_INVALID, "null argument");
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  *d_grads = o->g;
  *n_floats = o->n;
  o->grads_zero = false;  // the caller may write through the pointer from now on
  o->arena_exposed = true;
  o->sq_ready = false;
  return HB_OK;
}

extern "C" int hb_opt_grad_norm(hb_opt* o, float* out_norm) {
  HB_OPT_CHECK(o);
  if (!out_norm) return fail(HB_E_INVALID, "null argument");
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  TRY(opt_norm(o, ClipCfg{1.0f, o->tc.grad_clip}));
  return opt_read_norm(o, out_norm);
}

extern "C" int hb_opt_clip_grads(hb_opt* o, float max_norm, float* out_norm) {
  HB_OPT_CHECK(o);
  if (!(max_norm > 0.f)) return fail(HB_E_INVALID, "max_norm must be positive");
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  TRY(opt_norm(o, ClipCfg{1.0f, max_norm}));
  HIP_TRY(scale_inplace(o->g, o->n, o->scal + 2, o->model->ctx->stream()));
  o->sq_ready = false;
  return out_norm ? opt_read_norm(o, out_norm) : HB_OK;
}

extern "C" int hb_opt_update_weights(hb_opt* o, uint32_t t, float lr, float grad_scale) {
  HB_OPT_CHECK(o);
  if (t == 0) return fail(HB_E_INVALID, "t is 1-based");
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  return opt_update(o, t, lr, grad_scale, nullptr);
}

extern "C" int hb_opt_step(hb_opt* o, uint32_t step, float* out_norm) {
  HB_OPT_CHECK(o);
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  const hb_train_config& tc = o->tc;
  const float gsc = 1.0f / ((float)tc.accum_steps * tc.loss_scale);
  TRY(opt_norm(o, ClipCfg{gsc, tc.grad_clip}));
  TRY(opt_update(o, step + 1, learning_rate_f32(tc, step), 0.0f, o->scal + 1));
  return out_norm ? opt_read_norm(o, out_norm) : HB_OK;
}

extern "C" int hb_opt_download_layer(hb_opt* o, int layer, int which, float* wq, float* wk,
                                     float* wv, float* wo, float* w1, float* w3, float* w2,
                                     float* g1, float* g2) {
  HB_OPT_CHECK(o);
  const hb_model_config& c = o->model->cfg;
  if (layer < 0 || layer >= c.nlayers) return fail(HB_E_INVALID, "layer %d out of range", layer);
  float* a = opt_arena(o, which);
  if (!a) return fail(HB_E_INVALID, "which must be 0 (weights), 1 (m), 2 (v) or 3 (gradients)");
  float* w[9] = {wq, wk, wv, wo, w1, w3, w2, g1, g2};
  for (float* x : w)
    if (!x) return fail(HB_E_INVALID, "null output pointer");
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  const OptLayerOff& lo = o->lo[layer];
  const int d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden;
  const size_t n = lo.g2 + d - lo.wqkv;
  std::vector<float> host(n);
  hipStream_t st = o->model->ctx->stream();
  HIP_TRY(hipMemcpyAsync(host.data(), a + lo.wqkv, n * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  const float* b = host.data();
  unpack_host(b, d, q, d, 0, 0, wq);
  unpack_host(b, d, kv, d, q, 0, wk);
  unpack_host(b, d, kv, d, q + kv, 0, wv);
  unpack_host(b + (lo.wo - lo.wqkv), q, d, q, 0, 0, wo);
  unpack_host(b + (lo.w13 - lo.wqkv), d, h, d, 0, 1, w1);
  unpack_host(b + (lo.w13 - lo.wqkv), d, h, d, 2, 1, w3);
  unpack_host(b + (lo.w2 - lo.wqkv), d, h, h, 0, 2, w2);
  std::memcpy(g1, b + (lo.g1 - lo.wqkv), d * 4);
  std::memcpy(g2, b + (lo.g2 - lo.wqkv), d * 4);
  return HB_OK;
}

extern "C" int hb_opt_download_embed(hb_opt* o, int which, float* embed, float* gamma_final) {
  HB_OPT_CHECK(o);
  float* a = opt_arena(o, which);
  if (!a) return fail(HB_E_INVALID, "which must be 0 (weights), 1 (m), 2 (v) or 3 (gradients)");
  if (!embed || !gamma_final) return fail(HB_E_INVALID, "null output pointer");
  DeviceGuard g(o->device);
  TRY(opt_materialize(o));
  const hb_model_config& c = o->model->cfg;
  hipStream_t st = o->model->ctx->stream();
  HIP_TRY(hipMemcpyAsync(embed, a + o->embed_off, (size_t)c.vocab * c.dim * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(gamma_final, a + o->gf_off, c.dim * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return HB_OK;
}

// ---------------------------------------------------------------------------
// RSTK checkpoints (bin/train.rs:165-202)
// ---------------------------------------------------------------------------
namespace {
constexpr size_t RSTK_HDR = 28;

uint32_t le32(const unsigned char* p) {
  return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

int rstk_parse(const unsigned char* b, size_t n, hb_rstk_header* h) {
  if (n < RSTK_HDR || std::memcmp(b, "RSTK", 4) != 0)
    return fail(HB_E_INVALID, "not an RSTK checkpoint (bad magic or shorter than its header)");
  h->version = le32(b + 4);
  h->step = le32(b + 8);
  h->dim = le32(b + 12);
  h->nlayers = le32(b + 16);
  h->vocab = le32(b + 20);
  h->seq = le32(b + 24);
  if (h->version != 1) return fail(HB_E_INVALID, "RSTK version %u (only 1 is defined)", h->version);
  return HB_OK;
}

// fp32 values after the header for this config: embed, gamma_final, then per
// layer wq, wk, wv, wo, w1, w3, w2, gamma1, gamma2.
size_t rstk_floats(const hb_model_config& c) {
  const size_t d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden;
  const size_t per_layer = d * q + 2 * d * kv + q * d + 3 * d * h + 2 * d;
  return (size_t)c.vocab * d + d + (size_t)c.nlayers * per_layer;
}

struct MappedFile {
  const unsigned char* p = nullptr;
  size_t n = 0;
  ~MappedFile() {
    if (p) munmap((void*)p, n);
  }
};

int map_file(const char* path, MappedFile& mf) {
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(HB_E_INVALID, "cannot open %s", path);
  struct stat st {};
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return fail(HB_E_INVALID, "cannot stat %s (or it is empty)", path);
  }
  void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (p == MAP_FAILED) return fail(HB_E_INVALID, "cannot map %s", path);
  mf.p = (const unsigned char*)p;
  mf.n = (size_t)st.st_size;
  return HB_OK;
}

// The model's fp16 weights of one layer, widened and returned in the
// reference layouts (the inverse of hb_model_upload_layer's packing).
int model_download_layer(hb_model* m, int layer, std::vector<float> out[9]) {
  const hb_model_config& c = m->cfg;
  const LayerW& L = m->layers[layer];
  const int d = c.dim, q = c.q_dim, kv = c.kv_dim, h = c.hidden;
  hipStream_t st = m->ctx->stream();
  auto fetch = [&](const f16* src, size_t n, std::vector<float>& dst) -> int {
    std::vector<f16> tmp(n);
    HIP_TRY(hipMemcpyAsync(tmp.data(), src, n * 2, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    dst.resize(n);
    for (size_t i = 0; i < n; ++i) dst[i] = (float)tmp[i];
    return HB_OK;
  };
  std::vector<float> wqkv, wo, w13, w2;
  TRY(fetch(L.wqkv, (size_t)(q + 2 * kv) * d, wqkv));
  TRY(fetch(L.wo, (size_t)d * q, wo));
  TRY(fetch(L.w13, (size_t)2 * h * d, w13));
  TRY(fetch(L.w2, (size_t)d * h, w2));
  const size_t sz[9] = {(size_t)d * q, (size_t)d * kv, (size_t)d * kv, (size_t)q * d, (size_t)d * h,
                        (size_t)d * h, (size_t)d * h, (size_t)d, (size_t)d};
  for (int i = 0; i < 9; ++i) out[i].resize(sz[i]);
  unpack_host(wqkv.data(), d, q, d, 0, 0, out[0].data());
  unpack_host(wqkv.data(), d, kv, d, q, 0, out[1].data());
  unpack_host(wqkv.data(), d, kv, d, q + kv, 0, out[2].data());
  unpack_host(wo.data(), q, d, q, 0, 0, out[3].data());
  unpack_host(w13.data(), d, h, d, 0, 1, out[4].data());
  unpack_host(w13.data(), d, h, d, 2, 1, out[5].data());
  unpack_host(w2.data(), d, h, h, 0, 2, out[6].data());
  HIP_TRY(hipMemcpyAsync(out[7].data(), L.g1, d * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipMemcpyAsync(out[8].data(), L.g2, d * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return HB_OK;
}

struct FileCloser {
  FILE* f;
  ~FileCloser() {
    if (f) fclose(f);
  }
};
}  // namespace

extern "C" int hb_rstk_read_header(const char* path, hb_rstk_header* out) {
  HB_INJECT_CHECK();
  if (!path || !out) return fail(HB_E_INVALID, "null argument");
  FileCloser fc{fopen(path, "rb")};
  if (!fc.f) return fail(HB_E_INVALID, "cannot open %s", path);
  unsigned char b[RSTK_HDR];
  const size_t n = fread(b, 1, RSTK_HDR, fc.f);
  return rstk_parse(b, n, out);
}

extern "C" int hb_model_load_rstk(hb_model* m, hb_opt* opt, const char* path, uint32_t* out_step) {
  HB_INJECT_CHECK();
  if (!m || !path) return fail(HB_E_INVALID, "null argument");
  if (opt && opt->model != m) return fail(HB_E_INVALID, "optimizer belongs to another model");
  MappedFile mf;
  TRY(map_file(path, mf));
  hb_rstk_header h{};
  TRY(rstk_parse(mf.p, mf.n, &h));
  const hb_model_config& c = m->cfg;
  if ((int)h.dim != c.dim || (int)h.nlayers != c.nlayers || (int)h.vocab != c.vocab)
    return fail(HB_E_CONFIG, "checkpoint is dim %u / %u layers / vocab %u, the model %d / %d / %d",
                h.dim, h.nlayers, h.vocab, c.dim, c.nlayers, c.vocab);
  const size_t want = RSTK_HDR + 4 * rstk_floats(c);
  if (mf.n != want)
    return fail(HB_E_INVALID, "checkpoint has %zu bytes; this model's shapes give %zu", mf.n, want);
  const float* f = (const float*)(mf.p + RSTK_HDR);  // little-endian fp32, 4-byte aligned
  const size_t d = c.dim, q = c.q_dim, kv = c.kv_dim, hd = c.hidden;
  const float* embed = f;
  const float* gf = embed + (size_t)c.vocab * d;
  const float* p = gf + d;
  if (opt)
    TRY(hb_opt_upload_embed(opt, embed, gf));
  else
    TRY(hb_model_upload_embed(m, embed, gf));
  for (int l = 0; l < c.nlayers; ++l) {
    const float* w[9];
    const size_t sz[9] = {d * q, d * kv, d * kv, q * d, d * hd, d * hd, d * hd, d, d};
    for (int i = 0; i < 9; ++i) {
      w[i] = p;
      p += sz[i];
    }
    if (opt)
      TRY(hb_opt_upload_layer(opt, l, w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7], w[8]));
    else
      TRY(hb_model_upload_layer(m, l, w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7], w[8]));
  }
  if (out_step) *out_step = h.step;
  return HB_OK;
}

extern "C" int hb_model_save_rstk(hb_model* m, hb_opt* opt, uint32_t step, const char* path) {
  HB_INJECT_CHECK();
  if (!m || !path) return fail(HB_E_INVALID, "null argument");
  if (opt && opt->model != m) return fail(HB_E_INVALID, "optimizer belongs to another model");
  const hb_model_config& c = m->cfg;
  if (!opt) {
    if (!m->embed_uploaded) return fail(HB_E_STATE, "embedding not uploaded");
    for (const LayerW& L : m->layers)
      if (!L.uploaded) return fail(HB_E_STATE, "layer weights not uploaded");
  }
  DeviceGuard g(m->ctx->device);
  FileCloser fc{fopen(path, "wb")};
  if (!fc.f) return fail(HB_E_INVALID, "cannot create %s", path);
  unsigned char hdr[RSTK_HDR];
  std::memcpy(hdr, "RSTK", 4);
  const uint32_t vals[6] = {1u, step, (uint32_t)c.dim, (uint32_t)c.nlayers, (uint32_t)c.vocab,
                            (uint32_t)c.seq};
  for (int i = 0; i < 6; ++i)
    for (int b = 0; b < 4; ++b) hdr[4 + 4 * i + b] = (unsigned char)(vals[i] >> (8 * b));
  auto put = [&](const void* src, size_t bytes) -> int {
    if (fwrite(src, 1, bytes, fc.f) != bytes) return fail(HB_E_INVALID, "write to %s failed", path);
    return HB_OK;
  };
  TRY(put(hdr, RSTK_HDR));
  const size_t d = c.dim;
  std::vector<float> embed((size_t)c.vocab * d), gf(d);
  if (opt) {
    TRY(hb_opt_download_embed(opt, 0, embed.data(), gf.data()));
  } else {
    std::vector<f16> tmp(embed.size());
    hipStream_t st = m->ctx->stream();
    HIP_TRY(hipMemcpyAsync(tmp.data(), m->embed, tmp.size() * 2, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipMemcpyAsync(gf.data(), m->gamma_f, d * 4, hipMemcpyDeviceToHost, st));
    HIP_TRY(hipStreamSynchronize(st));
    for (size_t i = 0; i < tmp.size(); ++i) embed[i] = (float)tmp[i];
  }
  TRY(put(embed.data(), embed.size() * 4));
  TRY(put(gf.data(), d * 4));
  for (int l = 0; l < c.nlayers; ++l) {
    std::vector<float> w[9];
    if (opt) {
      const size_t q = c.q_dim, kv = c.kv_dim, h = c.hidden;
      const size_t sz[9] = {d * q, d * kv, d * kv, q * d, d * h, d * h, d * h, d, d};
      for (int i = 0; i < 9; ++i) w[i].resize(sz[i]);
      TRY(hb_opt_download_layer(opt, l, 0, w[0].data(), w[1].data(), w[2].data(), w[3].data(),
                                w[4].data(), w[5].data(), w[6].data(), w[7].data(), w[8].data()));
    } else {
      TRY(model_download_layer(m, l, w));
    }
    for (int i = 0; i < 9; ++i) TRY(put(w[i].data(), w[i].size() * 4));
  }
  if (fflush(fc.f) != 0) return fail(HB_E_INVALID, "write to %s failed", path);
  return HB_OK;
}

// ---------------------------------------------------------------------------
// data path and validation (data.rs, bin/train.rs:123-163)
// ---------------------------------------------------------------------------
static int forward_device_impl(hb_model* m, const uint32_t* d_tokens, const uint32_t* d_targets,
                               int B, int S, float* d_loss, float* d_logits, float* d_mean);

struct hb_tokens {
  int device = 0;
  uint16_t* d = nullptr;
  uint64_t n = 0;
};

extern "C" int hb_tokens_create(hb_ctx* ctx, const uint16_t* h, uint64_t n, hb_tokens** out) {
  HB_INJECT_CHECK();
  if (!ctx || !out || (!h && n)) return fail(HB_E_INVALID, "null argument");
  *out = nullptr;
  DeviceGuard g(ctx->device);
  hb_tokens* t = new hb_tokens();
  t->device = ctx->device;
  t->n = n;
  if (n) {
    hipError_t e = hipMalloc(&t->d, n * 2);
    if (e == hipSuccess) e = hipMemcpy(t->d, h, n * 2, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      if (t->d) (void)hipFree(t->d);
      delete t;
      return fail(e == hipErrorOutOfMemory ? HB_E_OOM : HB_E_DEVICE, "token stream of %llu ids: %s",
                  (unsigned long long)n, hipGetErrorString(e));
    }
  }
  *out = t;
  return HB_OK;
}

extern "C" int hb_tokens_open(hb_ctx* ctx, const char* path, hb_tokens** out) {
  HB_INJECT_CHECK();
  if (!ctx || !path || !out) return fail(HB_E_INVALID, "null argument");
  MappedFile mf;
  TRY(map_file(path, mf));
  if (mf.n % 2) return fail(HB_E_INVALID, "%s has an odd byte count (%zu)", path, mf.n);
  return hb_tokens_create(ctx, (const uint16_t*)mf.p, mf.n / 2, out);
}

extern "C" int hb_tokens_destroy(hb_tokens* t) {
  if (!t) return HB_OK;
  DeviceGuard g(t->device);
  if (t->d) (void)hipFree(t->d);
  delete t;
  return HB_OK;
}

extern "C" int hb_tokens_length(const hb_tokens* t, uint64_t* out) {
  HB_INJECT_CHECK();
  if (!t || !out) return fail(HB_E_INVALID, "null argument");
  *out = t->n;
  return HB_OK;
}

extern "C" int hb_validate(hb_model* m, const hb_tokens* val, const int32_t* token_bytes, int tb_len,
                           int steps, int batch, float* out_avg_loss, float* out_bpb,
                           double* out_nats, uint64_t* out_bytes) {
  HB_INJECT_CHECK();
  if (!m || !val) return fail(HB_E_INVALID, "null argument");
  if (steps < 1 || batch < 1) return fail(HB_E_INVALID, "steps and batch must be positive");
  if (token_bytes && tb_len < 1) return fail(HB_E_INVALID, "token_bytes needs tb_len >= 1");
  if (val->device != m->device) return fail(HB_E_INVALID, "token stream is on another device");
  const hb_model_config& c = m->cfg;
  const int S = c.seq;
  if (val->n < (uint64_t)S + 2)
    return fail(HB_E_INVALID, "%llu tokens: need at least seq + 2 = %d", (unsigned long long)val->n, S + 2);
  if (!weights_ready(m)) return fail(HB_E_STATE, "weights not uploaded");
  const int B = std::min(batch, steps);
  TRY(check_token_count(c, B, S));
  DeviceGuard g(m->ctx->device);
  TRY(ensure_workspace(m, (long)B * S, (long)B * S_pad_of(S)));
  Workspace& w = m->ws;
  hipStream_t st = m->ctx->stream();
  // totals (3 doubles) and the byte table in one scratch allocation
  const size_t tb_bytes = token_bytes ? (size_t)tb_len * 4 : 0;
  char* scratch = nullptr;
  HIP_TRY(hipMalloc(&scratch, 32 + tb_bytes));
  struct Free {
    char* p;
    ~Free() { (void)hipFree(p); }
  } fr{scratch};
  double* acc = (double*)scratch;
  int* tb = token_bytes ? (int*)(scratch + 32) : nullptr;
  HIP_TRY(hipMemsetAsync(acc, 0, 32, st));
  if (tb) HIP_TRY(hipMemcpyAsync(tb, token_bytes, tb_bytes, hipMemcpyHostToDevice, st));
  for (int vs = 0; vs < steps; vs += B) {
    const int nb = std::min(B, steps - vs);
    HIP_TRY(window_gather(val->d, val->n, (uint32_t)vs, nb, S, w.tok, w.tgt, st));
    TRY(forward_device_impl(m, w.tok, w.tgt, nb, S, w.loss, nullptr, nullptr));
    HIP_TRY(bpb_accum(w.loss, w.tgt, nb * S, tb, tb_len, acc, st));
  }
  double host[3];
  HIP_TRY(hipMemcpyAsync(host, acc, sizeof host, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  TRY(check_err_word(m->ctx));
  const double tokens = (double)steps * S;
  if (out_avg_loss) *out_avg_loss = (float)(host[0] / tokens);
  if (out_bpb) *out_bpb = host[2] > 0 ? (float)(host[1] / (0.69314718055994530942 * host[2])) : 0.0f;
  if (out_nats) *out_nats = host[1];
  if (out_bytes) *out_bytes = (uint64_t)host[2];
  return HB_OK;
}

// ---------------------------------------------------------------------------
// synthetic host inputs
// ---------------------------------------------------------------------------
template <class F>
static void parallel_for(uint64_t n, F f) {
  unsigned nt = std::min(16u, std::max(1u, std::thread::hardware_concurrency()));
  if (n < (1u << 16)) nt = 1;
  std::vector<std::thread> th;
  for (unsigned i = 0; i < nt; ++i)
    th.emplace_back([=] {
      const uint64_t a = n * i / nt, b = n * (i + 1) / nt;
      for (uint64_t j = a; j < b; ++j) f(j);
    });
  for (auto& t : th) t.join();
}

extern "C" int hb_synth_normal(uint64_t seed, uint64_t tensor_id, float std, uint64_t n, float* out) {
  HB_INJECT_CHECK();
  if (!out && n) return fail(HB_E_INVALID, "null out");
  const uint64_t key = hb_stream_key(seed, tensor_id);
  const float sc = hb_normal_scale(std);
  parallel_for(n, [=](uint64_t i) { out[i] = hb_normal_value(key, i, sc); });
  return HB_OK;
}

extern "C" int hb_synth_tokens(uint64_t seed, uint64_t stream, uint32_t vocab, uint64_t n,
                               uint32_t* out) {
  HB_INJECT_CHECK();
  if (!out && n) return fail(HB_E_INVALID, "null out");
  if (vocab == 0) return fail(HB_E_INVALID, "vocab must be positive");
  const uint64_t key = hb_stream_key(seed, stream);
  parallel_for(n, [=](uint64_t i) { out[i] = hb_token_value(key, i, vocab); });
  return HB_OK;
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
extern "C" int hb_model_reserve(hb_model* m, int B, int S) {
  HB_INJECT_CHECK();
  if (!m || B <= 0 || S <= 0) return fail(HB_E_INVALID, "bad argument");
  TRY(check_token_count(m->cfg, B, S));
  DeviceGuard g(m->ctx->device);
  return ensure_workspace(m, (long)B * S, (long)B * S_pad_of(S));
}

static int forward_enqueue(hb_model* m, const uint32_t* d_tokens, const uint32_t* d_targets, int B, int S,
                           float* d_loss, float* d_logits, float* d_mean, StageTimer* tm = nullptr);

// Allocates what forward_enqueue of (B, S) uses -- the workspace and the
// split-K scratch of the residual projections, for plain and two-term
// layers -- so that a capture of it allocates nothing.
static int forward_reserve(hb_model* m, int B, int S) {
  const hb_model_config& c = m->cfg;
  TRY(ensure_workspace(m, (long)B * S, (long)B * S_pad_of(S)));
  GemmScratch g;
  for (int f = 1; f <= (m->precise_layers > 0 ? 2 : 1); ++f) {
    TRY(residual_scratch(m, c.dim, B * S, f * c.q_dim, g));
    TRY(residual_scratch(m, c.dim, B * S, f * c.hidden, g));
  }
  return HB_OK;
}

// HB_NO_GRAPH=1 runs the forward and decode launches eagerly (for profiling
// individual launches).
static bool graphs_enabled() {
  const char* s = getenv("HB_NO_GRAPH");
  return !(s && s[0] == '1');
}

// The forward's launches depend only on the call's shape, pointers, softcap
// and split layers (and the addresses of the workspace, split-K scratch and
// RoPE table); the weights are read at run time. Repeated identical calls --
// a serving or benchmark loop -- replay one captured graph instead of ~7
// launches per layer, which is what bounds shallow or narrow models.
static int forward_device_impl(hb_model* m, const uint32_t* d_tokens, const uint32_t* d_targets,
                               int B, int S, float* d_loss, float* d_logits, float* d_mean) {
  const hb_model_config& c = m->cfg;
  if (B <= 0 || S <= 0 || S > c.seq) return fail(HB_E_INVALID, "need B >= 1 and 1 <= S <= seq (%d)", c.seq);
  TRY(check_token_count(c, B, S));
  if (!weights_ready(m)) return fail(HB_E_STATE, "weights not uploaded");
  if (!d_tokens) return fail(HB_E_INVALID, "null tokens");
  TRY(ensure_workspace(m, (long)B * S, (long)B * S_pad_of(S)));
  if (!graphs_enabled()) return forward_enqueue(m, d_tokens, d_targets, B, S, d_loss, d_logits, d_mean);
  auto key = [&]() {
    hb_model::FwdKey k;
    k.B = B; k.S = S; k.np = m->precise_layers; k.epoch = m->graph_epoch; k.softcap = c.softcap;
    k.tok = d_tokens; k.tgt = d_targets; k.loss = d_loss; k.logits = d_logits; k.mean = d_mean;
    k.ws = m->ws.base; k.splitk = m->splitk;
    return k;
  };
  hb_ctx* ctx = m->ctx;
  const hb_model::FwdKey k = key();
  if (m->fwd_exec && k == m->fwd_key) {
    HIP_TRY(hipGraphLaunch(m->fwd_exec, ctx->stream()));
    return HB_OK;
  }
  if (!(k == m->fwd_seen)) {  // first call of this shape: eager (it may allocate)
    TRY(forward_enqueue(m, d_tokens, d_targets, B, S, d_loss, d_logits, d_mean));
    m->fwd_seen = key();
    return HB_OK;
  }
  if (m->fwd_exec) (void)hipGraphExecDestroy(m->fwd_exec);
  if (m->fwd_graph) (void)hipGraphDestroy(m->fwd_graph);
  m->fwd_exec = nullptr;
  m->fwd_graph = nullptr;
  m->fwd_key = hb_model::FwdKey{};
  // everything the launches need is allocated before the capture starts
  TRY(forward_reserve(m, B, S));
  if (!(key() == k)) {  // the reservation moved the split-K scratch: capture on the next call
    m->fwd_seen = key();
    return forward_enqueue(m, d_tokens, d_targets, B, S, d_loss, d_logits, d_mean);
  }
  // the capture stream starts after the work already queued on the context stream
  HIP_TRY(hipStreamSynchronize(ctx->stream()));
  hipStream_t saved = ctx->user;
  ctx->user = ctx->capture;
  HIP_TRY(hipStreamBeginCapture(ctx->capture, hipStreamCaptureModeThreadLocal));
  const int r = forward_enqueue(m, d_tokens, d_targets, B, S, d_loss, d_logits, d_mean);
  hipGraph_t gr = nullptr;
  const hipError_t e = hipStreamEndCapture(ctx->capture, &gr);
  ctx->user = saved;
  if (r != HB_OK || e != hipSuccess) {
    if (gr) (void)hipGraphDestroy(gr);
    if (r != HB_OK) return r;
    return fail(HB_E_DEVICE, "forward graph capture failed: %s", hipGetErrorString(e));
  }
  m->fwd_graph = gr;
  HIP_TRY(hipGraphInstantiate(&m->fwd_exec, gr, nullptr, nullptr, 0));
  m->fwd_key = k;
  HIP_TRY(hipGraphLaunch(m->fwd_exec, ctx->stream()));
  return HB_OK;
}

static int forward_enqueue(hb_model* m, const uint32_t* d_tokens, const uint32_t* d_targets, int B, int S,
                           float* d_loss, float* d_logits, float* d_mean, StageTimer* tm) {
  const hb_model_config& c = m->cfg;
  const long T = (long)B * S;
  Workspace& w = m->ws;
  hipStream_t st = m->ctx->stream();
  HIP_TRY(embedding(m->embed, d_tokens, (int)T, c.dim, c.vocab, w.x, m->ctx->d_err, st));
  HB_MARK(tm, ST_EMBED);
  const KVTarget kv = scratch_kv(m, B, S);
  // Each layer leaves the next norm (the final one after the last layer) in xn.
  for (int l = 0; l < c.nlayers; ++l)
    TRY(run_layer(m, l, B, S, kv, nullptr, l > 0,
                  l + 1 < c.nlayers ? m->layers[l + 1].g1 : m->gamma_f, m->precise_layers, tm));
  if (tm) tm->layer = -1;
  float* logits = d_logits ? d_logits : w.logits;
  const int fl = m->precise_layers == c.nlayers ? 2 : 1;  // split final rows (run_layer)
  HIP_TRY(gemm_logits(m->embed, w.xn, c.vocab, (int)T, fl * c.dim, EpiLogits{logits, c.vocab, c.softcap}, st,
                      c.dim));
  HB_MARK(tm, ST_LOGITS);
  if (d_targets) {
    float* loss = d_loss ? d_loss : w.loss;
    HIP_TRY(cross_entropy(logits, d_targets, (int)T, c.vocab, loss, m->ctx->d_err, st));
    if (d_mean) HIP_TRY(mean_reduce(loss, (int)T, d_mean, st));
    HB_MARK(tm, ST_CE);
  }
  return HB_OK;
}

// forward_timed (layer.rs:821-1015) on the device: the launches of
// hb_forward_device, eager, with an event after each stage.
extern "C" int hb_forward_timed(hb_model* m, const uint32_t* d_tokens, const uint32_t* d_targets, int B,
                                int S, float* d_loss, float* d_mean, hb_forward_timings* out) {
  HB_INJECT_CHECK();
  if (!m || !out) return fail(HB_E_INVALID, "null argument");
  const hb_model_config& c = m->cfg;
  if (B <= 0 || S <= 0 || S > c.seq) return fail(HB_E_INVALID, "need B >= 1 and 1 <= S <= seq (%d)", c.seq);
  TRY(check_token_count(c, B, S));
  if (!weights_ready(m)) return fail(HB_E_STATE, "weights not uploaded");
  if (!d_tokens) return fail(HB_E_INVALID, "null tokens");
  DeviceGuard g(m->ctx->device);
  TRY(forward_reserve(m, B, S));
  hipStream_t st = m->ctx->stream();
  StageTimer tm{st};
  TRY(tm.mark(-1) == hipSuccess ? HB_OK : fail(HB_E_DEVICE, "event record failed"));
  TRY(forward_enqueue(m, d_tokens, d_targets, B, S, d_loss, nullptr, d_mean, &tm));
  HIP_TRY(hipStreamSynchronize(st));
  float stage[ST_COUNT] = {}, layer0 = 0.f;
  for (size_t i = 1; i < tm.ev.size(); ++i) {
    float ms = 0.f;
    HIP_TRY(hipEventElapsedTime(&ms, tm.ev[i - 1], tm.ev[i]));
    const int s_ = tm.tag[i].first, l = tm.tag[i].second;
    if (l == 0)
      layer0 += ms;
    else
      stage[s_] += ms;
  }
  float total = 0.f;
  HIP_TRY(hipEventElapsedTime(&total, tm.ev.front(), tm.ev.back()));
  *out = hb_forward_timings{};
  out->embedding_ms = stage[ST_EMBED];
  out->rmsnorm1_ms = stage[ST_NORM1];
  out->sdpa_qkv_ms = stage[ST_QKV];
  out->sdpa_attention_ms = stage[ST_ATTN];
  out->wo_ms = stage[ST_WO];
  out->residual_rmsnorm2_ms = stage[ST_WO_NORM];
  out->ffn_up_ms = stage[ST_FFN_UP];
  out->ffn_down_ms = stage[ST_FFN_DOWN];
  out->ffn_residual_norm_ms = stage[ST_FFN_NORM];
  out->logits_ms = stage[ST_LOGITS];
  out->cross_entropy_ms = stage[ST_CE];
  out->layer0_ms = layer0;
  out->total_ms = total;
  out->layers_summed = c.nlayers - 1;
  return check_err_word(m->ctx);
}

extern "C" int hb_forward_device(hb_model* m, const uint32_t* d_tokens, const uint32_t* d_targets,
                                 int B, int S, float* d_loss, float* d_logits, float* d_mean) {
  HB_INJECT_CHECK();
  if (!m) return fail(HB_E_INVALID, "null model");
  DeviceGuard g(m->ctx->device);
  return forward_device_impl(m, d_tokens, d_targets, B, S, d_loss, d_logits, d_mean);
}

static int check_ids(const uint32_t* ids, size_t n, int vocab, const char* what) {
  for (size_t i = 0; i < n; ++i)
    if (ids[i] >= (uint32_t)vocab)
      return fail(HB_E_INVALID, "%s[%zu] = %u out of range [0,%d)", what, i, ids[i], vocab);
  return HB_OK;
}

extern "C" int hb_forward(hb_model* m, const uint32_t* tokens, const uint32_t* targets, int B,
                          int S, float* per_pos_loss, float* logits, float* mean_loss) {
  HB_INJECT_CHECK();
  if (!m || !tokens) return fail(HB_E_INVALID, "null argument");
  if (B <= 0 || S <= 0 || S > m->cfg.seq) return fail(HB_E_INVALID, "need B >= 1 and 1 <= S <= seq (%d)", m->cfg.seq);
  TRY(check_token_count(m->cfg, B, S));
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  const size_t T = (size_t)B * S;
  TRY(check_ids(tokens, T, c.vocab, "tokens"));
  if (targets) TRY(check_ids(targets, T, c.vocab, "targets"));
  TRY(ensure_workspace(m, (long)T, (long)B * S_pad_of(S)));
  Workspace& w = m->ws;
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(w.tok, tokens, T * 4, hipMemcpyHostToDevice, st));
  if (targets) HIP_TRY(hipMemcpyAsync(w.tgt, targets, T * 4, hipMemcpyHostToDevice, st));
  TRY(forward_device_impl(m, w.tok, targets ? w.tgt : nullptr, B, S, w.loss, w.logits, w.mean));
  if (targets && per_pos_loss)
    HIP_TRY(hipMemcpyAsync(per_pos_loss, w.loss, T * 4, hipMemcpyDeviceToHost, st));
  if (targets && mean_loss) HIP_TRY(hipMemcpyAsync(mean_loss, w.mean, 4, hipMemcpyDeviceToHost, st));
  if (logits) HIP_TRY(hipMemcpyAsync(logits, w.logits, T * c.vocab * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return check_err_word(m->ctx);
}

// ---------------------------------------------------------------------------
// per-kernel entry points
// ---------------------------------------------------------------------------
extern "C" int hb_op_rmsnorm(hb_ctx* ctx, const float* x, const float* gamma, int T, int dim,
                             float eps, void* out, float* rms_inv) {
  HB_INJECT_CHECK();
  if (!ctx || !x || !gamma || !out) return fail(HB_E_INVALID, "null argument");
  if (T < 0 || dim <= 0 || dim % 4) return fail(HB_E_INVALID, "need T >= 0 and dim %% 4 == 0");
  if ((long)T * dim >= (1L << 31)) return fail(HB_E_INVALID, "T x dim exceeds 2^31 elements");
  DeviceGuard g(ctx->device);
  HIP_TRY(rmsnorm(x, dim, gamma, T, dim, eps, (f16*)out, rms_inv, ctx->stream()));
  return HB_OK;
}

extern "C" int hb_op_embedding(hb_model* m, const uint32_t* tok, int T, float* x) {
  HB_INJECT_CHECK();
  if (!m || !tok || !x) return fail(HB_E_INVALID, "null argument");
  if (!m->embed_uploaded) return fail(HB_E_STATE, "embedding not uploaded");
  if (T < 0 || (long)T * m->cfg.dim >= (1L << 31)) return fail(HB_E_INVALID, "need 0 <= T x dim < 2^31");
  DeviceGuard g(m->ctx->device);
  HIP_TRY(embedding(m->embed, tok, T, m->cfg.dim, m->cfg.vocab, x, m->ctx->d_err, m->ctx->stream()));
  return HB_OK;
}

extern "C" int hb_op_sdpa_fwd(hb_model* m, int layer, const void* xnorm, int B, int S, void* attn,
                              float* qkv_tap) {
  HB_INJECT_CHECK();
  if (!m || !xnorm || !attn) return fail(HB_E_INVALID, "null argument");
  if (layer < 0 || layer >= m->cfg.nlayers || !m->layers[layer].uploaded)
    return fail(HB_E_STATE, "layer %d not available", layer);
  if (B <= 0 || S <= 0 || S > m->cfg.seq) return fail(HB_E_INVALID, "bad B/S");
  TRY(check_token_count(m->cfg, B, S));
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  const int T = B * S, Sp = S_pad_of(S);
  TRY(ensure_workspace(m, T, (long)B * Sp));
  Workspace& w = m->ws;
  hipStream_t st = m->ctx->stream();
  const KVTarget kv = scratch_kv(m, B, S);
  EpiQKV e{};
  e.q_dim = c.q_dim; e.kv_dim = c.kv_dim; e.hd = c.hd; e.S = S; e.heads = c.heads;
  e.kv_heads = c.kv_heads; e.rope = m->rope; e.rope_ld = m->rope_len; e.d_pos = nullptr;
  e.q = w.q; e.q_rows = Sp;
  e.k = kv.k; e.k_bstride = kv.k_bstride; e.k_hstride = kv.k_hstride; e.v = nullptr;
  e.vt = w.vt; e.vt_ld = Sp; e.tap = qkv_tap;
  HIP_TRY(gemm_qkv(m->layers[layer].wqkv, (const f16*)xnorm, c.q_dim + 2 * c.kv_dim, T, c.dim, e, st));
  TRY(zero_vt_pad(m, w.vt, B, S, st));
  AttnPrefill a{};
  a.q = w.q; a.q_rows = Sp; a.k = kv.k; a.k_bstride = kv.k_bstride; a.k_hstride = kv.k_hstride;
  a.vt = w.vt; a.vt_ld = Sp; a.out = (f16*)attn; a.B = B; a.S = S; a.H = c.heads;
  a.KVH = c.kv_heads; a.hd = c.hd; a.scale = 1.0f / sqrtf((float)c.hd);
  HIP_TRY(attention_prefill(a, st));
  return HB_OK;
}

extern "C" int hb_op_wo_fwd(hb_model* m, int layer, const void* attn, const float* x, int T, float* x2) {
  HB_INJECT_CHECK();
  if (!m || !attn || !x || !x2) return fail(HB_E_INVALID, "null argument");
  if (layer < 0 || layer >= m->cfg.nlayers || !m->layers[layer].uploaded)
    return fail(HB_E_STATE, "layer %d not available", layer);
  if (T <= 0) return fail(HB_E_INVALID, "T must be positive");
  TRY(check_token_count(m->cfg, 1, T));
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  GemmScratch so;
  TRY(residual_scratch(m, c.dim, T, c.q_dim, so));
  HIP_TRY(gemm_residual(m->layers[layer].wo, (const f16*)attn, c.dim, T, c.q_dim,
                        EpiResidual{x, x2, c.dim, alpha_of(c)}, &so, m->ctx->stream()));
  return HB_OK;
}

extern "C" int hb_op_wo_fwd_noalloc(hb_model* m, int layer, const void* attn, const float* x, int T,
                                    float* x2) {
  HB_INJECT_CHECK();
  if (!m || !attn || !x || !x2) return fail(HB_E_INVALID, "null argument");
  if (layer < 0 || layer >= m->cfg.nlayers || !m->layers[layer].uploaded)
    return fail(HB_E_STATE, "layer %d not available", layer);
  if (T <= 0) return fail(HB_E_INVALID, "T must be positive");
  TRY(check_token_count(m->cfg, 1, T));
  const hb_model_config& c = m->cfg;
  const int splits = gemm_splits(c.dim, T, c.q_dim);
  if (splits > 1 && (size_t)splits * T * c.dim > NOALLOC_SCRATCH_FLOATS)
    return fail(HB_E_INVALID, "T=%d: %d K splits x %d x %d partial sums exceed the %zu-float no-alloc scratch", T,
                splits, T, c.dim, NOALLOC_SCRATCH_FLOATS);
  float* sp = scratch_of(m->ctx->device);
  if (!sp) return fail(HB_E_STATE, "no-alloc scratch not set up on device %d", m->ctx->device);
  DeviceGuard g(m->ctx->device);
  const GemmScratch so{sp, NOALLOC_SCRATCH_FLOATS, 256};
  hipStream_t st = m->ctx->stream();
  // ordered after the previous use of the array unless the stream is being
  // captured (a graph's replays are ordered by whoever launches them)
  const bool cap = capturing(m);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  hipEvent_t ev = g_scratch_ev[m->ctx->device];
  if (!cap) HIP_TRY(hipStreamWaitEvent(st, ev, 0));
  HIP_TRY(gemm_residual(m->layers[layer].wo, (const f16*)attn, c.dim, T, c.q_dim,
                        EpiResidual{x, x2, c.dim, alpha_of(c)}, &so, st));
  if (!cap) HIP_TRY(hipEventRecord(ev, st));
  return HB_OK;
}

extern "C" int hb_op_ffn_fused(hb_model* m, int layer, const void* x2norm, const float* x2, int T,
                               float* x_next, float* h13_tap, void* gate_out) {
  HB_INJECT_CHECK();
  if (!m || !x2norm || !x2 || !x_next) return fail(HB_E_INVALID, "null argument");
  if (layer < 0 || layer >= m->cfg.nlayers || !m->layers[layer].uploaded)
    return fail(HB_E_STATE, "layer %d not available", layer);
  if (T <= 0) return fail(HB_E_INVALID, "T must be positive");
  TRY(check_token_count(m->cfg, 1, T));
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  f16* gate = (f16*)gate_out;
  if (!gate) {
    TRY(ensure_workspace(m, T, std::max<long>(m->ws.cap_Tpad, 32)));
    gate = m->ws.gate;
  }
  hipStream_t st = m->ctx->stream();
  const LayerW& L = m->layers[layer];
  HIP_TRY(gemm_swiglu(L.w13, (const f16*)x2norm, 2 * c.hidden, T, c.dim, EpiSwiGLU{gate, h13_tap, c.hidden}, st));
  GemmScratch s2;
  TRY(residual_scratch(m, c.dim, T, c.hidden, s2));
  HIP_TRY(gemm_residual(L.w2, gate, c.dim, T, c.hidden, EpiResidual{x2, x_next, c.dim, alpha_of(c)}, &s2, st));
  return HB_OK;
}

extern "C" int hb_op_ffn_up(hb_model* m, int layer, const void* x2norm, int T, void* gate,
                            float* h13_tap) {
  HB_INJECT_CHECK();
  if (!m || !x2norm || !gate) return fail(HB_E_INVALID, "null argument");
  if (layer < 0 || layer >= m->cfg.nlayers || !m->layers[layer].uploaded)
    return fail(HB_E_STATE, "layer %d not available", layer);
  if (T <= 0) return fail(HB_E_INVALID, "T must be positive");
  TRY(check_token_count(m->cfg, 1, T));
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  HIP_TRY(gemm_swiglu(m->layers[layer].w13, (const f16*)x2norm, 2 * c.hidden, T, c.dim,
                      EpiSwiGLU{(f16*)gate, h13_tap, c.hidden}, m->ctx->stream()));
  return HB_OK;
}

extern "C" int hb_op_logits_ce(hb_model* m, const void* xf, const uint32_t* targets, int T,
                               float* logits, float* losses) {
  HB_INJECT_CHECK();
  if (!m || !xf) return fail(HB_E_INVALID, "null argument");
  if (!logits) return fail(HB_E_INVALID, "logits buffer required");
  if (!m->embed_uploaded) return fail(HB_E_STATE, "embedding not uploaded");
  if (T <= 0) return fail(HB_E_INVALID, "T must be positive");
  TRY(check_token_count(m->cfg, 1, T));
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  hipStream_t st = m->ctx->stream();
  HIP_TRY(gemm_logits(m->embed, (const f16*)xf, c.vocab, T, c.dim, EpiLogits{logits, c.vocab, c.softcap}, st));
  if (targets && losses)
    HIP_TRY(cross_entropy(logits, targets, T, c.vocab, losses, m->ctx->d_err, st));
  return HB_OK;
}

extern "C" int hb_op_gemm_nt(hb_ctx* ctx, const void* a, const void* b, float* cmat, int M, int N, int K) {
  HB_INJECT_CHECK();
  if (!ctx || !a || !b || !cmat) return fail(HB_E_INVALID, "null argument");
  if (M <= 0 || N <= 0 || K <= 0 || K % 64 || N % 4) return fail(HB_E_INVALID, "need K %% 64 == 0 and N %% 4 == 0");
  if (round64(std::max(M, N)) * std::max<long>(K, std::min(M, N)) >= (1L << 31))
    return fail(HB_E_INVALID, "M=%d N=%d K=%d exceeds the 2^31-element operand limit", M, N, K);
  DeviceGuard g(ctx->device);
  HIP_TRY(gemm_store((const f16*)b, (const f16*)a, N, M, K, cmat, ctx->stream()));
  return HB_OK;
}

// ---------------------------------------------------------------------------
// decode
// ---------------------------------------------------------------------------
namespace {

f16* cache_k(hb_kv* kv, int l) {
  const hb_model_config& c = kv->model->cfg;
  return kv->cache + (size_t)l * kv->B * 2 * c.kv_heads * kv->ctx_cap * c.hd;
}

KVTarget cache_target(hb_kv* kv, int l) {
  const hb_model_config& c = kv->model->cfg;
  KVTarget t{};
  t.k = cache_k(kv, l);
  t.k_hstride = (size_t)kv->ctx_cap * c.hd;
  t.k_bstride = 2 * (size_t)c.kv_heads * t.k_hstride;
  t.v = t.k + (size_t)c.kv_heads * t.k_hstride;
  t.v_bstride = t.k_bstride;
  t.v_hstride = t.k_hstride;
  if (l < kv->np) {  // same layout, one layer block per split layer
    t.k_lo = kv->lo_cache + (size_t)l * kv->B * 2 * c.kv_heads * kv->ctx_cap * c.hd;
    t.v_lo = t.k_lo + (size_t)c.kv_heads * t.k_hstride;
  }
  return t;
}

// Decode layer l < kv->np on two-term fp16 operands: separate norm, combine
// and GEMV launches on split rows (the fused prologues stage fp16 rows only).
int enqueue_decode_layer_split(hb_kv* kv, int l, const KVTarget& t, hipStream_t st) {
  hb_model* m = kv->model;
  const hb_model_config& c = m->cfg;
  const LayerW& L = m->layers[l];
  const int B = kv->B;
  const float alpha = alpha_of(c);
  HIP_TRY(rmsnorm(kv->x, c.dim, L.g1, B, c.dim, c.norm_eps, kv->xn, nullptr, st, true));
  EpiQKV e{};
  e.q_dim = c.q_dim; e.kv_dim = c.kv_dim; e.hd = c.hd; e.S = 1; e.heads = c.heads;
  e.kv_heads = c.kv_heads; e.rope = m->rope; e.rope_ld = m->rope_len; e.d_pos = kv->d_pos;
  e.q = kv->qd; e.q_rows = 1;
  e.k = t.k; e.k_bstride = t.k_bstride; e.k_hstride = t.k_hstride;
  e.v = t.v; e.v_bstride = t.v_bstride; e.v_hstride = t.v_hstride; e.vt = nullptr; e.vt_ld = 0;
  e.tap = nullptr;
  e.q_lo = kv->qd_lo; e.k_lo = t.k_lo; e.v_lo = t.v_lo;
  HIP_TRY(gemv_qkv(L.t_wqkv, kv->xn, nullptr, c.q_dim + 2 * c.kv_dim, B, c.dim, e, st, true));
  AttnDecode a{};
  a.q = kv->qd; a.k = t.k; a.v = t.v; a.bstride = t.k_bstride; a.hstride = t.k_hstride;
  a.d_pos = kv->d_pos; a.B = B; a.H = c.heads; a.KVH = c.kv_heads; a.hd = c.hd;
  a.ctx_max = kv->ctx_cap; a.nch = kv->nch; a.scale = 1.0f / sqrtf((float)c.hd); a.part_o = kv->part_o;
  a.part_ml = kv->part_ml; a.out = kv->attn;
  a.q_lo = kv->qd_lo; a.k_lo = t.k_lo; a.v_lo = t.v_lo;
  HIP_TRY(attention_decode(a, st));
  if (kv->nch > 1) HIP_TRY(attention_combine(a, st));
  HIP_TRY(gemv_residual(L.t_wo, kv->attn, nullptr, c.dim, B, c.q_dim, EpiResidual{kv->x, kv->x2, c.dim, alpha},
                        st, true));
  HIP_TRY(rmsnorm(kv->x2, c.dim, L.g2, B, c.dim, c.norm_eps, kv->xn, nullptr, st, true));
  HIP_TRY(gemv_swiglu(L.t_w13, kv->xn, nullptr, 2 * c.hidden, B, c.dim,
                      EpiSwiGLU{kv->gate, nullptr, c.hidden, true}, st, true));
  HIP_TRY(gemv_residual(L.t_w2, kv->gate, nullptr, c.dim, B, c.hidden, EpiResidual{kv->x2, kv->x, c.dim, alpha},
                        st, true));
  return HB_OK;
}

// One decode step over the kv->B sequences at position *d_pos. Launch shapes
// do not depend on the position, so the sequence can be captured once.
int enqueue_decode_step(hb_kv* kv, hipStream_t st) {
  hb_model* m = kv->model;
  const hb_model_config& c = m->cfg;
  const int B = kv->B;
  const float alpha = alpha_of(c);
  // Every RMSNorm runs inside the GEMV that consumes it while the staged rows
  // fit in LDS (B <= 3 at dim 4096): five launches per layer. Otherwise a
  // separate rmsnorm launch writes xn before each of those GEMVs.
  const bool fused = gemv_norm_fits(B, c.dim);
  // 8+ sequences: the separate norms write xn in the GEMVs' B-fragment order
  // (as the gate and the attention rows), one 1 KB operand block per k-step
  const bool xfrag = !fused && B >= 8 && c.dim % 32 == 0;
  auto prep_norm = [&](const float* x, const float* gamma, NormIn& n) -> hipError_t {
    n = NormIn{x, gamma, c.norm_eps};
    return fused ? hipSuccess
                 : rmsnorm(x, c.dim, gamma, B, c.dim, c.norm_eps, kv->xn, nullptr, st, false, xfrag);
  };
  HIP_TRY(embedding(m->embed, kv->d_tok, B, c.dim, c.vocab, kv->x, m->ctx->d_err, st));
  for (int l = 0; l < c.nlayers; ++l) {
    const LayerW& L = m->layers[l];
    const KVTarget t = cache_target(kv, l);
    if (l < kv->np) {
      TRY(enqueue_decode_layer_split(kv, l, t, st));
      continue;
    }
    NormIn n1, n2;
    HIP_TRY(prep_norm(kv->x, L.g1, n1));
    EpiQKV e{};
    e.q_dim = c.q_dim; e.kv_dim = c.kv_dim; e.hd = c.hd; e.S = 1; e.heads = c.heads;
    e.kv_heads = c.kv_heads; e.rope = m->rope; e.rope_ld = m->rope_len; e.d_pos = kv->d_pos;
    e.q = kv->qd; e.q_rows = 1;
    e.k = t.k; e.k_bstride = t.k_bstride; e.k_hstride = t.k_hstride;
    e.v = t.v; e.v_bstride = t.v_bstride; e.v_hstride = t.v_hstride; e.vt = nullptr; e.vt_ld = 0;
    e.tap = nullptr;
    HIP_TRY(gemv_qkv(L.t_wqkv, kv->xn, fused ? &n1 : nullptr, c.q_dim + 2 * c.kv_dim, B, c.dim, e, st,
                     false, xfrag));
    AttnDecode a{};
    a.q = kv->qd; a.k = t.k; a.v = t.v; a.bstride = t.k_bstride; a.hstride = t.k_hstride;
    a.d_pos = kv->d_pos; a.B = B; a.H = c.heads; a.KVH = c.kv_heads; a.hd = c.hd;
    a.ctx_max = kv->ctx_cap; a.nch = kv->nch; a.scale = 1.0f / sqrtf((float)c.hd); a.part_o = kv->part_o;
    a.part_ml = kv->part_ml; a.out = kv->attn;
    // 8+ sequences with one chunk: attention rows in Wo's B-fragment order
    // (as the gate for W2 below)
    a.out_frag = B >= 8 && kv->nch == 1 && c.q_dim % 32 == 0;
    HIP_TRY(attention_decode(a, st));
    if (kv->nch > 1 && !kv->attn_in_wo) HIP_TRY(attention_combine(a, st));
    const AttnIn ain{kv->part_o, kv->part_ml, kv->d_pos, c.heads, c.hd, kv->nch};
    HIP_TRY(gemv_residual(L.t_wo, kv->attn, kv->attn_in_wo ? &ain : nullptr, c.dim, B, c.q_dim,
                          EpiResidual{kv->x, kv->x2, c.dim, alpha}, st, false, a.out_frag));
    HIP_TRY(prep_norm(kv->x2, L.g2, n2));
    // 8+ sequences: the gate goes to W2 in B-fragment order (one 1 KB
    // operand block per k-step instead of B row pieces; 7B B = 16 decode
    // 5.94 -> 5.84 ms per step, B = 4 3.675 -> 3.694 ms, so not below 8)
    const bool frag = B >= 8 && c.hidden % 32 == 0;
    EpiSwiGLU sg{kv->gate, nullptr, c.hidden};
    sg.frag = frag;
    HIP_TRY(gemv_swiglu(L.t_w13, kv->xn, fused ? &n2 : nullptr, 2 * c.hidden, B, c.dim, sg, st, false, xfrag));
    HIP_TRY(gemv_residual(L.t_w2, kv->gate, nullptr, c.dim, B, c.hidden,
                          EpiResidual{kv->x2, kv->x, c.dim, alpha}, st, false, frag));
  }
  EpiLogits el{kv->logits, c.vocab, c.softcap};
  el.part_val = kv->amax_val;
  el.part_idx = kv->amax_idx;
  if (kv->np == c.nlayers) {  // every layer split: so are the final rows
    HIP_TRY(rmsnorm(kv->x, c.dim, m->gamma_f, B, c.dim, c.norm_eps, kv->xn, nullptr, st, true));
    HIP_TRY(gemv_logits(m->t_embed, kv->xn, nullptr, c.vocab, B, c.dim, el, st, true));
  } else {
    NormIn nf;
    HIP_TRY(prep_norm(kv->x, m->gamma_f, nf));
    HIP_TRY(gemv_logits(m->t_embed, kv->xn, fused ? &nf : nullptr, c.vocab, B, c.dim, el, st, false, xfrag));
  }
  HIP_TRY(argmax_reduce(kv->amax_val, kv->amax_idx, c.vocab / 16, B, kv->d_next, kv->d_tok,
                        kv->d_hist, kv->d_pos, kv->d_pos0, st));
  return HB_OK;
}


int launch_decode_step(hb_kv* kv) {
  hb_ctx* ctx = kv->model->ctx;
  if (!graphs_enabled()) return enqueue_decode_step(kv, ctx->stream());
  if (kv->exec && kv->graph_epoch != kv->model->graph_epoch) {
    HIP_TRY(hipStreamSynchronize(ctx->stream()));
    (void)hipGraphExecDestroy(kv->exec);
    (void)hipGraphDestroy(kv->graph);
    kv->exec = nullptr;
    kv->graph = nullptr;
  }
  if (!kv->exec) {
    HIP_TRY(hipStreamSynchronize(ctx->stream()));
    HIP_TRY(hipStreamBeginCapture(ctx->capture, hipStreamCaptureModeThreadLocal));
    int r = enqueue_decode_step(kv, ctx->capture);
    hipGraph_t gr = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->capture, &gr);
    if (r != HB_OK) {
      if (gr) (void)hipGraphDestroy(gr);
      return r;
    }
    if (e != hipSuccess) return fail(HB_E_DEVICE, "graph capture failed: %s", hipGetErrorString(e));
    kv->graph = gr;
    HIP_TRY(hipGraphInstantiate(&kv->exec, gr, nullptr, nullptr, 0));
    kv->graph_epoch = kv->model->graph_epoch;
  }
  HIP_TRY(hipGraphLaunch(kv->exec, ctx->stream()));
  return HB_OK;
}

}  // namespace

extern "C" int hb_kv_create(hb_model* m, int batch, int ctx_max, hb_kv** out) {
  HB_INJECT_CHECK();
  if (!m || !out) return fail(HB_E_INVALID, "null argument");
  *out = nullptr;
  if (batch < 1 || batch > 16) return fail(HB_E_INVALID, "batch must be in [1, 16] (got %d)", batch);
  if (ctx_max < 1) return fail(HB_E_INVALID, "ctx_max must be positive");
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  hb_kv* kv = new hb_kv();
  kv->model = m;
  kv->device = m->device;
  kv->B = batch;
  kv->ctx_max = ctx_max;
  kv->ctx_cap = (ctx_max + 63) & ~63;
  const AttnChunking ach = attn_decode_chunking(kv->ctx_cap, batch, m->cfg.heads);
  kv->nch = ach.n;
  kv->attn_in_wo = kv->nch > 1 && gemv_attn_fits(batch, m->cfg.q_dim, kv->nch);
  int r = ensure_rope(m, kv->ctx_cap);
  if (r != HB_OK) {
    delete kv;
    return r;
  }
  kv->cache_bytes = (size_t)c.nlayers * batch * 2 * c.kv_heads * kv->ctx_cap * c.hd * 2;
  hipError_t e = hipMalloc(&kv->cache, kv->cache_bytes);
  if (e != hipSuccess) {
    delete kv;
    return fail(e == hipErrorOutOfMemory ? HB_E_OOM : HB_E_DEVICE, "KV cache of %zu bytes: %s",
                kv->cache_bytes, hipGetErrorString(e));
  }
  kv->np = std::min(m->precise_layers, c.nlayers);
  if (kv->np > 0) {
    kv->lo_bytes = kv->cache_bytes / c.nlayers * kv->np;
    e = hipMalloc(&kv->lo_cache, kv->lo_bytes);
    if (e != hipSuccess) {
      (void)hipFree(kv->cache);
      delete kv;
      return fail(e == hipErrorOutOfMemory ? HB_E_OOM : HB_E_DEVICE, "KV low parts of %zu bytes: %s",
                  kv->lo_bytes, hipGetErrorString(e));
    }
  }
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += align256(bytes);
    return o;
  };
  const size_t B = batch;
  const size_t o_pos = take(4), o_pos0 = take(4), o_tok = take(B * 4), o_next = take(B * 4);
  const size_t o_hist = take((size_t)kv->ctx_cap * B * 4);
  const size_t o_x = take(B * c.dim * 4), o_x2 = take(B * c.dim * 4);
  const size_t o_logits = take(B * c.vocab * 4);
  const size_t o_po = take(B * c.heads * kv->nch * c.hd * 4), o_pml = take(B * c.heads * kv->nch * 8);
  const size_t o_aval = take(B * (c.vocab / 16) * 4), o_aidx = take(B * (c.vocab / 16) * 4);
  // xn, attn and gate hold split rows [B, 2K] in split layers
  // xn and attn also hold B-fragment order (16 row slots of K halves) at 8+
  // sequences, gate at any batch: each at least 16 rows
  const size_t rows16 = std::max<size_t>(2 * B, 16);
  const size_t o_xn = take(rows16 * c.dim * 2), o_qd = take(B * c.q_dim * 2), o_attn = take(rows16 * c.q_dim * 2);
  // gate: split rows [B][2*hidden], or (B >= 8) B-fragment order over 16 row slots
  const size_t o_gate = take(rows16 * c.hidden * 2), o_qdlo = take(B * c.q_dim * 2);
  char* sb = nullptr;
  e = hipMalloc(&sb, off);
  if (e != hipSuccess) {
    (void)hipFree(kv->cache);
    if (kv->lo_cache) (void)hipFree(kv->lo_cache);
    delete kv;
    return fail(HB_E_OOM, "decode buffers: %s", hipGetErrorString(e));
  }
  kv->sbase = sb;
  kv->d_pos = (int*)(sb + o_pos);
  kv->d_pos0 = (int*)(sb + o_pos0);
  kv->d_tok = (uint32_t*)(sb + o_tok);
  kv->d_next = (uint32_t*)(sb + o_next);
  kv->d_hist = (uint32_t*)(sb + o_hist);
  kv->x = (float*)(sb + o_x);
  kv->x2 = (float*)(sb + o_x2);
  kv->logits = (float*)(sb + o_logits);
  kv->part_o = (float*)(sb + o_po);
  kv->part_ml = (float*)(sb + o_pml);
  kv->amax_val = (float*)(sb + o_aval);
  kv->amax_idx = (int*)(sb + o_aidx);
  kv->xn = (f16*)(sb + o_xn);
  kv->qd = (f16*)(sb + o_qd);
  kv->attn = (f16*)(sb + o_attn);
  kv->gate = (f16*)(sb + o_gate);
  kv->qd_lo = (f16*)(sb + o_qdlo);
  hipStream_t st = m->ctx->stream();
  e = hipMemsetAsync(sb, 0, off, st);
  if (e == hipSuccess) e = fill_f16_zero(kv->cache, kv->cache_bytes / 2, st);
  if (e == hipSuccess && kv->lo_cache) e = fill_f16_zero(kv->lo_cache, kv->lo_bytes / 2, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    (void)hipFree(kv->cache);
    if (kv->lo_cache) (void)hipFree(kv->lo_cache);
    (void)hipFree(sb);
    delete kv;
    return fail(HB_E_DEVICE, "KV init: %s", hipGetErrorString(e));
  }
  *out = kv;
  return HB_OK;
}

extern "C" int hb_kv_destroy(hb_kv* kv) {
  if (!kv) return HB_OK;
  DeviceGuard g(kv->device);
  (void)hipDeviceSynchronize();
  if (kv->exec) (void)hipGraphExecDestroy(kv->exec);
  if (kv->graph) (void)hipGraphDestroy(kv->graph);
  (void)hipFree(kv->cache);
  if (kv->lo_cache) (void)hipFree(kv->lo_cache);
  (void)hipFree(kv->sbase);
  delete kv;
  return HB_OK;
}

extern "C" int hb_kv_reset(hb_kv* kv) {
  HB_INJECT_CHECK();
  if (!kv) return fail(HB_E_INVALID, "null kv");
  DeviceGuard g(kv->model->ctx->device);
  HIP_TRY(set_int(kv->d_pos, 0, kv->model->ctx->stream()));
  HIP_TRY(hipStreamSynchronize(kv->model->ctx->stream()));
  kv->len = 0;
  return HB_OK;
}

extern "C" int hb_kv_length(hb_kv* kv, int* out) {
  HB_INJECT_CHECK();
  if (!kv || !out) return fail(HB_E_INVALID, "null argument");
  *out = kv->len;
  return HB_OK;
}

extern "C" int hb_kv_bytes(hb_kv* kv, uint64_t* out) {
  HB_INJECT_CHECK();
  if (!kv || !out) return fail(HB_E_INVALID, "null argument");
  *out = kv->cache_bytes + kv->lo_bytes;
  return HB_OK;
}

extern "C" int hb_prefill(hb_model* m, hb_kv* kv, const uint32_t* tokens, int S, float* h_logits,
                          uint32_t* h_next) {
  HB_INJECT_CHECK();
  if (!m || !kv || !tokens) return fail(HB_E_INVALID, "null argument");
  if (kv->model != m) return fail(HB_E_INVALID, "kv cache belongs to another model");
  if (kv->len != 0) return fail(HB_E_STATE, "prefill needs an empty cache (length %d)", kv->len);
  if (S < 1 || S > kv->ctx_max) return fail(HB_E_INVALID, "S must be in [1, ctx_max]");
  TRY(check_token_count(m->cfg, kv->B, S));
  if (!weights_ready(m)) return fail(HB_E_STATE, "weights not uploaded");
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  const int B = kv->B;
  const long T = (long)B * S;
  TRY(check_ids(tokens, T, c.vocab, "tokens"));
  TRY(ensure_rope(m, kv->ctx_cap));
  TRY(ensure_workspace(m, T, (long)B * S_pad_of(S), kv->np > 0));
  TRY(ensure_decode_weights(m));
  Workspace& w = m->ws;
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(w.tok, tokens, T * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(embedding(m->embed, w.tok, (int)T, c.dim, c.vocab, w.x, m->ctx->d_err, st));
  for (int l = 0; l < c.nlayers; ++l)
    TRY(run_layer(m, l, B, S, cache_target(kv, l), nullptr, l > 0,
                  l + 1 < c.nlayers ? m->layers[l + 1].g1 : nullptr, kv->np));
  // Last position of each sequence -> logits and greedy token.
  const bool sf = kv->np == c.nlayers;  // every layer split: so are the final rows
  HIP_TRY(rmsnorm(w.x + (size_t)(S - 1) * c.dim, (long)S * c.dim, m->gamma_f, B, c.dim, c.norm_eps,
                  kv->xn, nullptr, st, sf));
  EpiLogits el{kv->logits, c.vocab, c.softcap};
  el.part_val = kv->amax_val;
  el.part_idx = kv->amax_idx;
  HIP_TRY(gemv_logits(m->t_embed, kv->xn, nullptr, c.vocab, B, c.dim, el, st, sf));
  HIP_TRY(argmax_reduce(kv->amax_val, kv->amax_idx, c.vocab / 16, B, kv->d_next, nullptr, nullptr,
                        nullptr, nullptr, st));
  HIP_TRY(set_int(kv->d_pos, S, st));
  if (h_logits) HIP_TRY(hipMemcpyAsync(h_logits, kv->logits, (size_t)B * c.vocab * 4, hipMemcpyDeviceToHost, st));
  if (h_next) HIP_TRY(hipMemcpyAsync(h_next, kv->d_next, (size_t)B * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  TRY(check_err_word(m->ctx));
  kv->len = S;
  return HB_OK;
}

extern "C" int hb_decode_step(hb_model* m, hb_kv* kv, const uint32_t* tokens, float* h_logits,
                              uint32_t* h_next) {
  HB_INJECT_CHECK();
  if (!m || !kv || !tokens) return fail(HB_E_INVALID, "null argument");
  if (kv->model != m) return fail(HB_E_INVALID, "kv cache belongs to another model");
  if (kv->len >= kv->ctx_max) return fail(HB_E_STATE, "KV cache full (%d positions)", kv->ctx_max);
  if (!weights_ready(m)) return fail(HB_E_STATE, "weights not uploaded");
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  TRY(check_ids(tokens, kv->B, c.vocab, "tokens"));
  TRY(ensure_decode_weights(m));
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(kv->d_tok, tokens, (size_t)kv->B * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(set_int(kv->d_pos0, kv->len, st));
  TRY(launch_decode_step(kv));
  if (h_logits) HIP_TRY(hipMemcpyAsync(h_logits, kv->logits, (size_t)kv->B * c.vocab * 4, hipMemcpyDeviceToHost, st));
  if (h_next) HIP_TRY(hipMemcpyAsync(h_next, kv->d_next, (size_t)kv->B * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  TRY(check_err_word(m->ctx));
  kv->len += 1;
  return HB_OK;
}

extern "C" int hb_decode_greedy(hb_model* m, hb_kv* kv, const uint32_t* first, int nsteps,
                                uint32_t* h_out) {
  HB_INJECT_CHECK();
  if (!m || !kv || !first) return fail(HB_E_INVALID, "null argument");
  if (kv->model != m) return fail(HB_E_INVALID, "kv cache belongs to another model");
  if (nsteps < 0 || kv->len + nsteps > kv->ctx_max)
    return fail(HB_E_STATE, "%d steps from length %d exceed ctx_max %d", nsteps, kv->len, kv->ctx_max);
  if (!weights_ready(m)) return fail(HB_E_STATE, "weights not uploaded");
  DeviceGuard g(m->ctx->device);
  const hb_model_config& c = m->cfg;
  TRY(check_ids(first, kv->B, c.vocab, "first tokens"));
  TRY(ensure_decode_weights(m));
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(kv->d_tok, first, (size_t)kv->B * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(set_int(kv->d_pos0, kv->len, st));
  for (int i = 0; i < nsteps; ++i) TRY(launch_decode_step(kv));
  if (h_out && nsteps)
    HIP_TRY(hipMemcpyAsync(h_out, kv->d_hist, (size_t)nsteps * kv->B * 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  TRY(check_err_word(m->ctx));
  kv->len += nsteps;
  return HB_OK;
}

// ---------------------------------------------------------------------------
// training: forward with kept activations + backward into the gradient arena
// ---------------------------------------------------------------------------

namespace {


// Transposed copies of every matrix, rebuilt after any weight write.
int train_weights(hb_model* m) {
  const hb_model_config& c = m->cfg;
  TrainState* ts = m->train;
  const long d = c.dim, h = c.hidden, q = c.q_dim, qkv = c.q_dim + 2L * c.kv_dim;
  const long Vp = round64(c.vocab);
  hipStream_t st = m->ctx->stream();
  if (!ts->wtbase) {
    const size_t per = align256(d * qkv * 2) + align256(q * d * 2) + align256(2 * h * d * 2) +
                       align256(h * d * 2);
    const size_t bytes = per * c.nlayers + align256(d * Vp * 2);
    char* base = nullptr;
    HIP_TRY(hipMalloc(&base, bytes));
    ts->wtbase = base;
    size_t off = 0;
    for (int l = 0; l < c.nlayers; ++l) {
      ts->wqkvT.push_back((f16*)(base + off)); off += align256(d * qkv * 2);
      ts->woT.push_back((f16*)(base + off)); off += align256(q * d * 2);
      ts->w13T.push_back((f16*)(base + off)); off += align256(2 * h * d * 2);
      ts->w2T.push_back((f16*)(base + off)); off += align256(h * d * 2);
    }
    ts->eT = (f16*)(base + off);
    m->wt_stale = true;
  }
  if (!m->wt_stale) return HB_OK;
  for (int l = 0; l < c.nlayers; ++l) {
    const LayerW& L = m->layers[l];
    HIP_TRY(transpose_f16(L.wqkv, (int)qkv, (int)d, (int)d, 0, ts->wqkvT[l], (int)qkv, 0, 1, st));
    HIP_TRY(transpose_f16(L.wo, (int)d, (int)q, (int)q, 0, ts->woT[l], (int)d, 0, 1, st));
    HIP_TRY(transpose_f16(L.w13, (int)(2 * h), (int)d, (int)d, 0, ts->w13T[l], (int)(2 * h), 0, 1, st));
    HIP_TRY(transpose_f16(L.w2, (int)d, (int)h, (int)h, 0, ts->w2T[l], (int)d, 0, 1, st));
  }
  HIP_TRY(transpose_f16(m->embed, c.vocab, (int)d, (int)d, 0, ts->eT, (int)Vp, 0, 1, st));
  m->wt_stale = false;
  return HB_OK;
}

// Activation + scratch arena for (B, S), zero-filled whenever the shape
// changes so that every padding row and column starts at zero.
int train_buffers(hb_model* m, int B, int S) {
  const hb_model_config& c = m->cfg;
  TrainState* ts = m->train;
  if (ts->abase && ts->B == B && ts->S == S) return HB_OK;
  const long T = (long)B * S, Sp = round64(S), Tp = round64(T), Vp = round64(c.vocab);
  const long d = c.dim, h = c.hidden, q = c.q_dim, kv = c.kv_dim, qkv = q + 2 * kv, V = c.vocab;
  const long qh = (long)B * c.heads * Sp * c.hd, kvh = (long)B * c.kv_heads * Sp * c.hd;
  const long qrows = (long)B * c.heads * Sp;  // per-query attention statistics
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += align256(bytes);
    return o;
  };
  struct ActOff {
    size_t x, x2, h13, xn, x2n, q, k, v, attn, gate, lse;
  };
  std::vector<ActOff> ao(c.nlayers);
  for (auto& a : ao) {
    a.x = take(T * d * 4); a.x2 = take(T * d * 4); a.h13 = take(T * 2 * h * 4);
    a.xn = take(T * d * 2); a.x2n = take(T * d * 2); a.q = take(qh * 2); a.k = take(kvh * 2);
    a.v = take(kvh * 2); a.attn = take(T * q * 2); a.gate = take(T * h * 2); a.lse = take(qrows * 4);
  }
  const size_t o_xL = take(T * d * 4), o_logits = take(T * V * 4), o_loss = take(T * 4),
               o_mean = take(4), o_xf = take(T * d * 2), o_tok = take(T * 4), o_tgt = take(T * 4);
  const size_t o_dy = take(T * d * 4), o_dx2 = take(T * d * 4), o_dtmp = take(T * d * 4),
               o_rinv = take(T * 4), o_part = take(rmsnorm_backward_part_floats(c.dim) * 4);
  const size_t o_D = take(qrows * 4);
  const long actw = std::max(std::max(h, d), q);
  const size_t o_d16 = take(T * d * 2), o_d16T = take(d * Tp * 2), o_dh = take(T * 2 * h * 2),
               o_dhT = take(2 * h * Tp * 2), o_actT = take(actw * Tp * 2), o_dqkv = take(T * qkv * 2),
               o_dqkvT = take(qkv * Tp * 2), o_dl = take(T * Vp * 2), o_dlT = take(V * Tp * 2);
  const size_t o_dA = take(qh * 2), o_dAT = take(qh * 2), o_qT = take(qh * 2), o_kT = take(kvh * 2),
               o_vt = take(kvh * 2);
  hipStream_t st = m->ctx->stream();
  if (off > ts->abytes) {
    HIP_TRY(hipStreamSynchronize(st));
    if (ts->abase) HIP_TRY(hipFree(ts->abase));
    ts->abase = nullptr;
    ts->abytes = 0;
    HIP_TRY(hipMalloc(&ts->abase, off));
    ts->abytes = off;
  }
  char* b = (char*)ts->abase;
  ts->act.resize(c.nlayers);
  for (int l = 0; l < c.nlayers; ++l) {
    LayerAct& A = ts->act[l];
    const ActOff& a = ao[l];
    A.x = (float*)(b + a.x); A.x2 = (float*)(b + a.x2); A.h13 = (float*)(b + a.h13);
    A.xn = (f16*)(b + a.xn); A.x2n = (f16*)(b + a.x2n); A.q = (f16*)(b + a.q); A.k = (f16*)(b + a.k);
    A.v = (f16*)(b + a.v); A.attn = (f16*)(b + a.attn); A.gate = (f16*)(b + a.gate);
    A.lse = (float*)(b + a.lse);
  }
  ts->xL = (float*)(b + o_xL); ts->logits = (float*)(b + o_logits); ts->loss = (float*)(b + o_loss);
  ts->mean = (float*)(b + o_mean); ts->xf = (f16*)(b + o_xf); ts->tok = (uint32_t*)(b + o_tok);
  ts->tgt = (uint32_t*)(b + o_tgt);
  ts->dy = (float*)(b + o_dy); ts->dx2 = (float*)(b + o_dx2); ts->dtmp = (float*)(b + o_dtmp);
  ts->rinv = (float*)(b + o_rinv); ts->part = (float*)(b + o_part);
  ts->Drow = (float*)(b + o_D);
  ts->d16 = (f16*)(b + o_d16); ts->d16T = (f16*)(b + o_d16T); ts->dh = (f16*)(b + o_dh);
  ts->dhT = (f16*)(b + o_dhT); ts->actT = (f16*)(b + o_actT); ts->dqkv = (f16*)(b + o_dqkv);
  ts->dqkvT = (f16*)(b + o_dqkvT); ts->dl = (f16*)(b + o_dl); ts->dlT = (f16*)(b + o_dlT);
  ts->dA = (f16*)(b + o_dA); ts->dAT = (f16*)(b + o_dAT); ts->qT = (f16*)(b + o_qT);
  ts->kT = (f16*)(b + o_kT); ts->vt = (f16*)(b + o_vt);
  HIP_TRY(fill_f16_zero((f16*)b, off / 2, st));
  ts->B = B;
  ts->S = S;
  return HB_OK;
}

// forward_ws (full_model.rs:187-247) keeping every layer's activations.
int train_forward(hb_model* m, int B, int S) {
  const hb_model_config& c = m->cfg;
  TrainState* ts = m->train;
  hipStream_t st = m->ctx->stream();
  const int T = B * S, Sp = (int)round64(S);
  const int qkv = c.q_dim + 2 * c.kv_dim;
  const float alpha = alpha_of(c);
  const size_t khs = (size_t)Sp * c.hd, kbs = (size_t)c.kv_heads * khs;
  ts->softcap = c.softcap;
  HIP_TRY(embedding(m->embed, ts->tok, T, c.dim, c.vocab, ts->act[0].x, m->ctx->d_err, st));
  for (int l = 0; l < c.nlayers; ++l) {
    const LayerW& L = m->layers[l];
    const LayerAct& A = ts->act[l];
    float* xout = l + 1 < c.nlayers ? ts->act[l + 1].x : ts->xL;
    HIP_TRY(rmsnorm(A.x, c.dim, L.g1, T, c.dim, c.norm_eps, A.xn, nullptr, st));
    EpiQKV e{};
    e.q_dim = c.q_dim; e.kv_dim = c.kv_dim; e.hd = c.hd; e.S = S; e.heads = c.heads;
    e.kv_heads = c.kv_heads; e.rope = m->rope; e.rope_ld = m->rope_len; e.d_pos = nullptr;
    e.q = A.q; e.q_rows = Sp;
    e.k = A.k; e.k_bstride = kbs; e.k_hstride = khs;
    e.v = A.v; e.v_bstride = kbs; e.v_hstride = khs;
    e.vt = ts->vt; e.vt_ld = Sp; e.tap = nullptr;
    HIP_TRY(gemm_qkv(L.wqkv, A.xn, qkv, T, c.dim, e, st));
    AttnPrefill a{};
    a.q = A.q; a.q_rows = Sp; a.k = A.k; a.k_bstride = kbs; a.k_hstride = khs;
    a.vt = ts->vt; a.vt_ld = Sp; a.out = A.attn; a.B = B; a.S = S; a.H = c.heads;
    a.KVH = c.kv_heads; a.hd = c.hd; a.scale = 1.0f / sqrtf((float)c.hd); a.lse = A.lse;
    HIP_TRY(attention_prefill(a, st));
    GemmScratch so, s2;
    TRY(residual_scratch(m, c.dim, T, c.q_dim, so));
    HIP_TRY(gemm_residual_norm(L.wo, A.attn, c.dim, T, c.q_dim, EpiResidual{A.x, A.x2, c.dim, alpha},
                               NormOut{L.g2, c.norm_eps, A.x2n}, &so, st));
    HIP_TRY(gemm_swiglu(L.w13, A.x2n, 2 * c.hidden, T, c.dim, EpiSwiGLU{A.gate, A.h13, c.hidden}, st));
    TRY(residual_scratch(m, c.dim, T, c.hidden, s2));
    HIP_TRY(gemm_residual(L.w2, A.gate, c.dim, T, c.hidden, EpiResidual{A.x2, xout, c.dim, alpha}, &s2, st));
  }
  HIP_TRY(rmsnorm(ts->xL, c.dim, m->gamma_f, T, c.dim, c.norm_eps, ts->xf, nullptr, st));
  HIP_TRY(gemm_logits(m->embed, ts->xf, c.vocab, T, c.dim, EpiLogits{ts->logits, c.vocab, ts->softcap}, st));
  HIP_TRY(cross_entropy(ts->logits, ts->tgt, T, c.vocab, ts->loss, m->ctx->d_err, st));
  HIP_TRY(mean_reduce(ts->loss, T, ts->mean, st));
  return HB_OK;
}

// Attention backward of one layer (kernels/sdpa_bwd.rs:46-161): the fused
// kernels (attention_bwd.hip) recompute P from Q, K and the forward's
// log-sum-exp, with the operands they read as MFMA A fragments transposed
// first (K^T, and the rep = heads/kv_heads query heads of a group stacked as
// [hd][rep*Sp] for Q^T and dO^T), and write dQ, dK, dV with RoPE^-1 into the
// dQKV rows and their transpose.
int attention_backward(hb_model* m, const LayerAct& A, int B, int S) {
  const hb_model_config& c = m->cfg;
  TrainState* ts = m->train;
  hipStream_t st = m->ctx->stream();
  const int Sp = (int)round64(S), T = B * S, Tp = (int)round64(T);
  const int Z = B * c.kv_heads, rep = c.heads / c.kv_heads, Rq = rep * Sp, hd = c.hd;
  const size_t khs = (size_t)Sp * hd, qzs = (size_t)Rq * hd;
  HIP_TRY(transpose_f16(A.k, Sp, hd, hd, khs, ts->kT, Sp, khs, Z, st));
  HIP_TRY(transpose_f16(A.q, Rq, hd, hd, qzs, ts->qT, Rq, qzs, Z, st));
  HIP_TRY(transpose_f16(ts->dA, Rq, hd, hd, qzs, ts->dAT, Rq, qzs, Z, st));
  AttnBwd p{};
  p.q = A.q; p.dO = ts->dA; p.k = A.k; p.v = A.v; p.qT = ts->qT; p.dOT = ts->dAT; p.kT = ts->kT;
  p.lse = A.lse; p.D = ts->Drow;
  p.B = B; p.S = S; p.Sp = Sp; p.H = c.heads; p.KVH = c.kv_heads; p.hd = hd;
  p.scale = 1.0f / sqrtf((float)hd);
  p.dqkv = ts->dqkv; p.dqkvT = ts->dqkvT; p.ld = c.q_dim + 2 * c.kv_dim; p.tld = Tp;
  p.q_dim = c.q_dim; p.kv_dim = c.kv_dim; p.rope = m->rope; p.rope_ld = m->rope_len;
  (void)T;
  HIP_TRY(attention_backward_fused(p, st));
  return HB_OK;
}

// backward_ws (full_model.rs:250-331) with layer::backward_into
// (layer.rs:1606-1858) per layer, accumulating into the optimizer's fp32
// gradient arena (packed order, element for element like the fp16 weights).
int train_backward_impl(hb_model* m, hb_opt* o, int B, int S, float loss_scale) {
  const hb_model_config& c = m->cfg;
  TrainState* ts = m->train;
  hipStream_t st = m->ctx->stream();
  const int T = B * S, Tp = (int)round64(T), Vp = (int)round64(c.vocab), Sp = (int)round64(S);
  const int d = c.dim, h = c.hidden, q = c.q_dim, qkv = c.q_dim + 2 * c.kv_dim;
  const float alpha = alpha_of(c);
  float* g = o->g;
  // every gradient element is written below: onto zeros, store instead of add
  const bool acc = !o->grads_zero;
  // sums of squares of the written gradient (for the norm): one slot per
  // weight-gradient tile and per 256 gamma entries; the embedding is summed
  // after its scatter-add
  const long gblk = (d + 255) / 256;
  const long cap = c.nlayers * (gemm_wgrad_max_tiles(h, d) + gemm_wgrad_max_tiles(d, 2 * h) +
                                gemm_wgrad_max_tiles(q, d) + gemm_wgrad_max_tiles(d, qkv) + 2 * gblk) +
                   gblk;
  if (o->sq_cap < cap) {
    HIP_TRY(hipStreamSynchronize(st));
    if (o->sq_slots) HIP_TRY(hipFree(o->sq_slots));
    o->sq_slots = nullptr;
    o->sq_cap = 0;
    HIP_TRY(hipMalloc(&o->sq_slots, cap * sizeof(float)));
    o->sq_cap = cap;
  }
  if (!o->sq_embed) HIP_TRY(hipMalloc(&o->sq_embed, SUMSQ_BLOCKS * sizeof(double)));
  o->sq_ready = false;
  long ns = 0;
  // slots for the next writer (at most `need`), checked before its launch
  auto slot = [&](long need) -> float* { return ns + need <= o->sq_cap ? o->sq_slots + ns : nullptr; };
  float* sq = nullptr;
  int nt = 0;
  // head: dlogits, dX of the tied embedding, dE, final norm. |dlogits| <= gs
  // = loss_scale/S while most entries are p*gs with p ~ 1/vocab: in fp16 they
  // would sit at or below the subnormal range (the reference keeps this head
  // in fp32, full_model.rs:250-331). So dl is stored as fp16(dl * f) with the
  // power of two f that puts gs near 2^14, and both products divide f back
  // out in their epilogues (exact).
  const float gs = loss_scale / (float)S;
  int fexp = 0;
  (void)frexpf(16384.0f / gs, &fexp);
  const float f = ldexpf(1.0f, fexp - 1), inv_f = ldexpf(1.0f, 1 - fexp);
  HIP_TRY(ce_backward(ts->logits, ts->tgt, T, c.vocab, Vp, gs * f, ts->softcap, ts->dl, st));
  HIP_TRY(transpose_f16(ts->dl, T, c.vocab, Vp, 0, ts->dlT, Tp, 0, 1, st));
  GemmScratch se;
  TRY(residual_scratch(m, d, T, Vp, se, 512));
  HIP_TRY(gemm_store_split(ts->eT, ts->dl, d, T, Vp, ts->dtmp, &se, st, inv_f));
  HIP_TRY(transpose_f16(ts->xf, T, d, d, 0, ts->actT, Tp, 0, 1, st));
  HIP_TRY(gemm_wgrad(ts->actT, ts->dlT, d, c.vocab, Tp, g + o->embed_off, d, acc, st, inv_f));
  if (!(sq = slot(gblk))) return fail(HB_E_STATE, "gradient norm slots exhausted");
  HIP_TRY(rmsnorm_backward(ts->dtmp, ts->xL, m->gamma_f, nullptr, T, d, c.norm_eps, ts->dy, ts->rinv,
                           ts->part, g + o->gf_off, acc, st, sq));
  ns += gblk;
  for (int l = c.nlayers - 1; l >= 0; --l) {
    const LayerW& L = m->layers[l];
    const LayerAct& A = ts->act[l];
    const OptLayerOff& go = o->lo[l];
    // FFN: x_out = x2 + alpha * W2 (silu(W1 x2n) * W3 x2n)
    HIP_TRY(cast_transpose(ts->dy, T, d, alpha, ts->d16, ts->d16T, Tp, st));
    HIP_TRY(gemm_silu_bwd(ts->w2T[l], ts->d16, h, T, d, EpiSiluBwd{A.h13, ts->dh, h}, st));
    HIP_TRY(transpose_f16(ts->dh, T, 2 * h, 2 * h, 0, ts->dhT, Tp, 0, 1, st));
    GemmScratch s13, sqkv;
    TRY(residual_scratch(m, d, T, 2 * h, s13, 512));
    HIP_TRY(gemm_store_split(ts->w13T[l], ts->dh, d, T, 2 * h, ts->dtmp, &s13, st));
    HIP_TRY(transpose_f16(A.gate, T, h, h, 0, ts->actT, Tp, 0, 1, st));
    if (!(sq = slot(gemm_wgrad_max_tiles(h, d)))) return fail(HB_E_STATE, "gradient norm slots exhausted");
    HIP_TRY(gemm_wgrad(ts->actT, ts->d16T, h, d, Tp, g + go.w2, h, acc, st, 1.0f, sq, &nt));
    ns += nt;
    HIP_TRY(transpose_f16(A.x2n, T, d, d, 0, ts->actT, Tp, 0, 1, st));
    if (!(sq = slot(gemm_wgrad_max_tiles(d, 2 * h)))) return fail(HB_E_STATE, "gradient norm slots exhausted");
    HIP_TRY(gemm_wgrad(ts->actT, ts->dhT, d, 2 * h, Tp, g + go.w13, d, acc, st, 1.0f, sq, &nt));
    ns += nt;
    if (!(sq = slot(gblk))) return fail(HB_E_STATE, "gradient norm slots exhausted");
    HIP_TRY(rmsnorm_backward(ts->dtmp, A.x2, L.g2, ts->dy, T, d, c.norm_eps, ts->dx2, ts->rinv, ts->part,
                             g + go.g2, acc, st, sq));
    ns += gblk;
    // attention: x2 = x + alpha * Wo attn(x n)
    HIP_TRY(cast_transpose(ts->dx2, T, d, alpha, ts->d16, ts->d16T, Tp, st));
    HIP_TRY(gemm_heads(ts->woT[l], ts->d16, q, T, d, EpiHeads{ts->dA, S, c.heads, c.hd, Sp}, st));
    HIP_TRY(transpose_f16(A.attn, T, q, q, 0, ts->actT, Tp, 0, 1, st));
    if (!(sq = slot(gemm_wgrad_max_tiles(q, d)))) return fail(HB_E_STATE, "gradient norm slots exhausted");
    HIP_TRY(gemm_wgrad(ts->actT, ts->d16T, q, d, Tp, g + go.wo, q, acc, st, 1.0f, sq, &nt));
    ns += nt;
    TRY(attention_backward(m, A, B, S));
    TRY(residual_scratch(m, d, T, qkv, sqkv, 512));
    HIP_TRY(gemm_store_split(ts->wqkvT[l], ts->dqkv, d, T, qkv, ts->dtmp, &sqkv, st));
    HIP_TRY(transpose_f16(A.xn, T, d, d, 0, ts->actT, Tp, 0, 1, st));
    if (!(sq = slot(gemm_wgrad_max_tiles(d, qkv)))) return fail(HB_E_STATE, "gradient norm slots exhausted");
    HIP_TRY(gemm_wgrad(ts->actT, ts->dqkvT, d, qkv, Tp, g + go.wqkv, d, acc, st, 1.0f, sq, &nt));
    ns += nt;
    if (!(sq = slot(gblk))) return fail(HB_E_STATE, "gradient norm slots exhausted");
    HIP_TRY(rmsnorm_backward(ts->dtmp, A.x, L.g1, ts->dx2, T, d, c.norm_eps, ts->dy, ts->rinv, ts->part,
                             g + go.g1, acc, st, sq));
    ns += gblk;
  }
  HIP_TRY(embedding_backward(ts->dy, ts->tok, T, d, c.vocab, g + o->embed_off, st));
  HIP_TRY(grad_sumsq(g + o->embed_off, (size_t)c.vocab * d, o->sq_embed, st));
  o->sq_n = ns;
  return HB_OK;
}

// Runs the backward and settles the arena's state flags. The per-tile sums of
// squares stand for the arena only while nobody else can write it: once
// hb_opt_grad_arena has handed out the raw pointer, a caller's later write
// would be missing from them, so the norm then takes the full pass. A
// backward that fails part way leaves a partly written arena: one that held
// zeros is marked for clearing by its next consumer, so no stale half-result
// is read as a gradient.
int train_backward(hb_model* m, hb_opt* o, int B, int S, float loss_scale) {
  const bool was_zero = o->grads_zero;
  o->sq_ready = false;
  const int r = train_backward_impl(m, o, B, S, loss_scale);
  if (r != HB_OK) {
    o->grads_zero = o->lazy_zero = was_zero;
    return r;
  }
  o->sq_ready = !o->arena_exposed;
  o->grads_zero = false;
  o->lazy_zero = false;  // every element was stored
  return HB_OK;
}

int check_loss_scale(float loss_scale) {
  if (!(loss_scale > 0.f) || !std::isfinite(loss_scale)) return fail(HB_E_INVALID, "loss_scale must be positive");
  return HB_OK;
}

// Checks a training forward of (B, S) and brings the transposed weights and
// the (B, S) buffers up to date.
int train_prepare_model(hb_model* m, int B, int S) {
  const hb_model_config& c = m->cfg;
  if (B <= 0 || S <= 0 || S > c.seq) return fail(HB_E_INVALID, "need B >= 1 and 1 <= S <= seq (%d)", c.seq);
  if (!weights_ready(m)) return fail(HB_E_STATE, "weights not uploaded");
  if (c.dim > 8192) return fail(HB_E_CONFIG, "training needs dim <= 8192");
  const long T = (long)B * S, Sp = round64(S);
  if (round64(T) * std::max<long>(c.vocab, 2L * c.hidden) >= (1L << 31) ||
      (long)c.heads / c.kv_heads * Sp * Sp >= (1L << 31) || (long)B * c.kv_heads > 65535)
    return fail(HB_E_INVALID, "B=%d S=%d too large for one training call", B, S);
  if (!m->train) m->train = new TrainState();
  m->train->kept = false;
  TRY(train_weights(m));
  TRY(train_buffers(m, B, S));
  return HB_OK;
}

int train_prepare(hb_model* m, hb_opt* o, int B, int S, float loss_scale) {
  if (!o || o->model != m) return fail(HB_E_INVALID, "optimizer belongs to another model");
  TRY(check_loss_scale(loss_scale));
  return train_prepare_model(m, B, S);
}

// ForwardResult's host views (full_model.rs:73-81) of the training forward
// just run, copied out in the reference's layouts.
int train_forward_views(hb_model* m, int B, int S, const hb_forward_result* r) {
  const hb_model_config& c = m->cfg;
  TrainState* ts = m->train;
  hipStream_t st = m->ctx->stream();
  const size_t T = (size_t)B * S, TV = T * c.vocab, Td = T * c.dim;
  const bool want_cap = r->logits_capped && ts->softcap > 0.f;
  const size_t need = (r->dlogits ? TV : 0) + (want_cap ? TV : 0) + (r->x_prenorm ? Td : 0) +
                      (r->x_final ? Td : 0) + T;
  if (need > ts->views_floats) {
    HIP_TRY(hipStreamSynchronize(st));
    if (ts->views) HIP_TRY(hipFree(ts->views));
    ts->views = nullptr;
    ts->views_floats = 0;
    HIP_TRY(hipMalloc(&ts->views, need * 4));
    ts->views_floats = need;
  }
  float* p = ts->views;
  auto take = [&](bool want, size_t n) {
    float* q = want ? p : nullptr;
    p += want ? n : 0;
    return q;
  };
  float* d_dl = take(r->dlogits != nullptr, TV);
  float* d_cap = take(want_cap, TV);
  float* d_pre = take(r->x_prenorm != nullptr, Td);
  float* d_fin = take(r->x_final != nullptr, Td);
  float* d_rinv = take(true, T);
  if (d_dl || d_cap)
    HIP_TRY(ce_grad_views(ts->logits, ts->tgt, (int)T, c.vocab, 1.0f / (float)S, ts->softcap, d_dl, d_cap, st));
  // the forward's own rms_inv (same kernel, same reduction order)
  HIP_TRY(rmsnorm(ts->xL, c.dim, m->gamma_f, (int)T, c.dim, c.norm_eps, ts->xf, d_rinv, st));
  if (d_pre || d_fin)
    HIP_TRY(final_norm_views(ts->xL, m->gamma_f, d_rinv, B, S, c.dim, d_pre, d_fin, st));
  auto down = [&](float* h, const float* d, size_t n) -> hipError_t {
    return h && d ? hipMemcpyAsync(h, d, n * 4, hipMemcpyDeviceToHost, st) : hipSuccess;
  };
  HIP_TRY(down(r->dlogits, d_dl, TV));
  HIP_TRY(down(r->logits_capped, d_cap, TV));
  HIP_TRY(down(r->x_prenorm, d_pre, Td));
  HIP_TRY(down(r->x_final, d_fin, Td));
  HIP_TRY(down(r->rms_inv_final, d_rinv, T));
  return HB_OK;
}

}  // namespace

extern "C" int hb_forward_backward_device(hb_model* m, hb_opt* o, const uint32_t* d_tokens,
                                          const uint32_t* d_targets, int B, int S, float loss_scale,
                                          float* d_loss, float* d_mean) {
  HB_INJECT_CHECK();
  if (!m || !o || !d_tokens || !d_targets) return fail(HB_E_INVALID, "null argument");
  DeviceGuard g(m->ctx->device);
  TRY(train_prepare(m, o, B, S, loss_scale));
  TrainState* ts = m->train;
  hipStream_t st = m->ctx->stream();
  const size_t T = (size_t)B * S;
  HIP_TRY(hipMemcpyAsync(ts->tok, d_tokens, T * 4, hipMemcpyDeviceToDevice, st));
  HIP_TRY(hipMemcpyAsync(ts->tgt, d_targets, T * 4, hipMemcpyDeviceToDevice, st));
  TRY(train_forward(m, B, S));
  TRY(train_backward(m, o, B, S, loss_scale));
  if (d_loss) HIP_TRY(hipMemcpyAsync(d_loss, ts->loss, T * 4, hipMemcpyDeviceToDevice, st));
  if (d_mean) HIP_TRY(hipMemcpyAsync(d_mean, ts->mean, 4, hipMemcpyDeviceToDevice, st));
  return HB_OK;
}

extern "C" int hb_train_forward(hb_model* m, const uint32_t* tokens, const uint32_t* targets, int B, int S,
                                float* per_pos_loss, float* mean_loss, const hb_forward_result* out) {
  HB_INJECT_CHECK();
  if (!m || !tokens || !targets) return fail(HB_E_INVALID, "null argument");
  DeviceGuard g(m->ctx->device);
  TRY(train_prepare_model(m, B, S));
  const size_t T = (size_t)B * S;
  TRY(check_ids(tokens, T, m->cfg.vocab, "tokens"));
  TRY(check_ids(targets, T, m->cfg.vocab, "targets"));
  TrainState* ts = m->train;
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(ts->tok, tokens, T * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ts->tgt, targets, T * 4, hipMemcpyHostToDevice, st));
  TRY(train_forward(m, B, S));
  if (out) TRY(train_forward_views(m, B, S, out));
  if (per_pos_loss) HIP_TRY(hipMemcpyAsync(per_pos_loss, ts->loss, T * 4, hipMemcpyDeviceToHost, st));
  if (mean_loss) HIP_TRY(hipMemcpyAsync(mean_loss, ts->mean, 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  TRY(check_err_word(m->ctx));
  ts->kept = true;
  return HB_OK;
}

extern "C" int hb_train_backward(hb_model* m, hb_opt* o, float loss_scale) {
  HB_INJECT_CHECK();
  if (!m || !o) return fail(HB_E_INVALID, "null argument");
  if (o->model != m) return fail(HB_E_INVALID, "optimizer belongs to another model");
  TRY(check_loss_scale(loss_scale));
  TrainState* ts = m->train;
  if (!ts || !ts->kept) return fail(HB_E_STATE, "no kept training forward (call hb_train_forward first)");
  DeviceGuard g(m->ctx->device);
  ts->kept = false;
  // the weights may have been written since the forward: the backward uses
  // the current ones, as the reference's backward takes `weights` afresh
  TRY(train_weights(m));
  TRY(train_backward(m, o, ts->B, ts->S, loss_scale));
  HIP_TRY(hipStreamSynchronize(m->ctx->stream()));
  return check_err_word(m->ctx);
}

extern "C" int hb_forward_backward(hb_model* m, hb_opt* o, const uint32_t* tokens,
                                   const uint32_t* targets, int B, int S, float loss_scale,
                                   float* per_pos_loss, float* mean_loss) {
  HB_INJECT_CHECK();
  if (!m || !o || !tokens || !targets) return fail(HB_E_INVALID, "null argument");
  DeviceGuard g(m->ctx->device);
  TRY(train_prepare(m, o, B, S, loss_scale));
  const size_t T = (size_t)B * S;
  TRY(check_ids(tokens, T, m->cfg.vocab, "tokens"));
  TRY(check_ids(targets, T, m->cfg.vocab, "targets"));
  TrainState* ts = m->train;
  hipStream_t st = m->ctx->stream();
  HIP_TRY(hipMemcpyAsync(ts->tok, tokens, T * 4, hipMemcpyHostToDevice, st));
  HIP_TRY(hipMemcpyAsync(ts->tgt, targets, T * 4, hipMemcpyHostToDevice, st));
  TRY(train_forward(m, B, S));
  TRY(train_backward(m, o, B, S, loss_scale));
  if (per_pos_loss) HIP_TRY(hipMemcpyAsync(per_pos_loss, ts->loss, T * 4, hipMemcpyDeviceToHost, st));
  if (mean_loss) HIP_TRY(hipMemcpyAsync(mean_loss, ts->mean, 4, hipMemcpyDeviceToHost, st));
  HIP_TRY(hipStreamSynchronize(st));
  return check_err_word(m->ctx);
}
