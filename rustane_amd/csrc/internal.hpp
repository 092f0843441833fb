// Internal launcher API shared by the kernel translation units and the C ABI.
#pragma once
#include "common.hpp"
#include "epilogue.hpp"

namespace hb {

// ---- prefill GEMM (gemm.hip, gemm_qkv.hip, gemm_ffn.hip, gemm_train.hip) ----
// Scratch for split-K partial sums (fp32); see gemm_splits.
struct GemmScratch {
  float* p;
  size_t floats;
  int wgs = 256;  // workgroups the split count aims for (gemm_splits)
};
constexpr int GEMM_MAX_SPLITS = 8;
// One product, or n of them with operands wbs / xbs halfs apart (blockIdx.z).
struct GemmBatch {
  int n = 1;
  size_t wbs = 0, xbs = 0;
};
// Number of K splits the residual GEMM uses for this shape when given scratch
// (1 = none), aiming at wgs workgroups; it needs splits * T * N floats.
int gemm_splits(int N, int T, int K, int wgs = 256);
// The same for gemm_residual_norm, which may use 256x128 tiles (*wide) for
// long reductions; it needs splits * T * N floats too.
int gemm_norm_splits(int N, int T, int K, int wgs, bool* wide);
hipError_t gemm_store(const f16* W, const f16* X, int N, int T, int K, float* C, hipStream_t st);
// kw (the residual, SwiGLU and QKV projections): 0 for plain X rows of K
// halves; for split X rows (common.hpp) K = 2 * kw with kw the weights' row
// length.
hipError_t gemm_residual(const f16* W, const f16* X, int N, int T, int K, const EpiResidual& e,
                         const GemmScratch* scr, hipStream_t st, int kw = 0);
// Residual projection followed by the RMSNorm of its output rows into xn
// (fused into the split-K reduction when the shape splits).
struct NormOut {
  const float* gamma;
  float eps;
  f16* xn;             // [T, N], or split rows [T, 2N]
  bool split = false;
};
// mid (nullable): an event recorded after the projection, before the
// reduction / norm launch (a timed forward's stage boundary).
hipError_t gemm_residual_norm(const f16* W, const f16* X, int N, int T, int K, const EpiResidual& e,
                              const NormOut& no, const GemmScratch* scr, hipStream_t st, int kw = 0,
                              hipEvent_t mid = nullptr);
hipError_t gemm_swiglu(const f16* W, const f16* X, int N, int T, int K, const EpiSwiGLU& e,
                       hipStream_t st, int kw = 0);
hipError_t gemm_logits(const f16* W, const f16* X, int N, int T, int K, const EpiLogits& e,
                       hipStream_t st, int kw = 0);
hipError_t gemm_qkv(const f16* W, const f16* X, int N, int T, int K, const EpiQKV& e,
                    hipStream_t st, int kw = 0);

// Training products (the epilogues are documented in epilogue.hpp). All take
// K % 64 == 0; token-dimension (K = tokens) operands are zero-padded to it.
// C = X W^T (fp32 store), split over K into scr when the shape leaves CUs idle
// (gemm_splits), as the residual GEMMs are.
hipError_t gemm_store_split(const f16* W, const f16* X, int N, int T, int K, float* C,
                            const GemmScratch* scr, hipStream_t st, float scale = 1.0f);
// Weight gradient g[t, f] (+)= sum_k X[t,k] W[f,k]: accumulate (EpiAccum) or,
// when the arena is known to be zero, store. With short K (<= 1024 tokens) the
// fp32 read-modify-write dominates: 128x128 tiles (two per CU) when there are
// enough of them.
// With sq_out, one sum of squares of the written gradient per output tile
// goes to sq_out[0 .. *sq_tiles) (gemm_wgrad_max_tiles bounds the count).
hipError_t gemm_wgrad(const f16* W, const f16* X, int N, int T, int K, float* g, int ld,
                      bool accumulate, hipStream_t st, float scale = 1.0f, float* sq_out = nullptr,
                      int* sq_tiles = nullptr);
inline long gemm_wgrad_max_tiles(int N, int T) { return (long)((N + 127) / 128) * ((T + 127) / 128); }
hipError_t gemm_silu_bwd(const f16* W, const f16* X, int N, int T, int K, const EpiSiluBwd& e,
                         hipStream_t st);
hipError_t gemm_heads(const f16* W, const f16* X, int N, int T, int K, const EpiHeads& e,
                      hipStream_t st);

// ---- decode GEMV (gemv.hip): rows of X are the B <= 16 sequences ----
// W arguments are decode copies in fragment-tiled order (tile_decode); N is a
// multiple of 16 and K of 32.
hipError_t tile_decode(const f16* W, f16* Wt, int N, int K, hipStream_t st);
// Input RMSNorm done inside the GEMV (nin != NULL): the B rows of x [B, K]
// fp32 are normalised with gamma [K] and staged in LDS; X is then unused.
struct NormIn {
  const float* x;
  const float* gamma;
  float eps;
};
constexpr int GEMV_NORM_MAXB = 8;
constexpr size_t GEMV_NORM_LDS = 32768;  // bytes of staged fp16 rows
bool gemv_norm_fits(int B, int K);
// Decode-attention chunk combine done inside the Wo GEMV (ain != NULL): the
// B x H heads' chunk partials of attention_decode are combined
// into the fp16 attention rows [B, H*hd], staged in LDS; X is then unused.
struct AttnIn {
  const float* part_o;   // [B][H][nch][hd]
  const float* part_ml;  // [B][H][nch][2]
  const int* d_pos;      // chunks attn_chunks_valid(*d_pos, nch) hold keys
  int H, hd, nch;
};
constexpr int GEMV_ATTN_MAXCH = 8;  // B * nch limit of the in-GEMV combine
bool gemv_attn_fits(int B, int K, int nch);
// split: X rows are split rows [B, 2K] (common.hpp), read from memory (no
// prologue); the weights are still [N, K].
// xfrag: X in B-fragment order (EpiSwiGLU::frag), no prologue.
hipError_t gemv_residual(const f16* Wt, const f16* X, const AttnIn* ain, int N, int B, int K,
                         const EpiResidual& e, hipStream_t st, bool split = false, bool xfrag = false);
hipError_t gemv_swiglu(const f16* Wt, const f16* X, const NormIn* nin, int N, int B, int K,
                       const EpiSwiGLU& e, hipStream_t st, bool split = false,
                       bool xfrag = false);
hipError_t gemv_logits(const f16* Wt, const f16* X, const NormIn* nin, int N, int B, int K,
                       const EpiLogits& e, hipStream_t st, bool split = false,
                       bool xfrag = false);
hipError_t gemv_qkv(const f16* Wt, const f16* X, const NormIn* nin, int N, int B, int K,
                    const EpiQKV& e, hipStream_t st, bool split = false,
                       bool xfrag = false);
hipError_t gemv_store(const f16* Wt, const f16* X, int N, int B, int K, float* C, hipStream_t st);
// Greedy token from the logits GEMV's argmax partials ([B][nblk] each). With
// tok != NULL it also feeds the token back (tok, hist row pos - *d_pos0) and
// advances *d_pos.
hipError_t argmax_reduce(const float* pval, const int* pidx, int nblk, int B, uint32_t* next,
                         uint32_t* tok, uint32_t* hist, int* d_pos, const int* d_pos0,
                         hipStream_t st);

// ---- attention (attention.hip) ----
struct AttnPrefill {
  const f16* q;  // [B][H][q_rows][hd]
  int q_rows;
  const f16* k;  // rows [s][hd] at k + b*k_bstride + kvh*k_hstride
  size_t k_bstride, k_hstride;
  const f16* vt;  // [B][KVH][hd][vt_ld]
  int vt_ld;
  f16* out;  // [B*S][H*hd], or split rows [B*S][2*H*hd] when q_lo is set
  int B, S, H, KVH, hd;
  float scale;  // 1/sqrt(hd)
  // Two-term fp16 inputs (common.hpp): low parts of q, k and vt in the same
  // layouts, all set or all NULL.
  const f16 *q_lo = nullptr, *k_lo = nullptr, *vt_lo = nullptr;
  // Training: per-query log-sum-exp of the scaled scores in log2 units,
  // lse[(b*H + h)*q_rows + s] = log2(sum_t exp2(sc[s,t] * scale * log2 e)),
  // for the fused backward. NULL: not written.
  float* lse = nullptr;
};
hipError_t attention_prefill(const AttnPrefill& p, hipStream_t st);

// Fused attention backward (kernels/sdpa_bwd.rs:46-161) for one layer of the
// training forward: P is recomputed from Q, K and the forward's log-sum-exp,
// so no score matrix is stored. Two launches:
//   dQ:     per (2 query blocks, head, sequence): D = rowsum(P * dP), then
//           dS = P (dP - D) scale and dQ = dS K, RoPE^-1
//   dK, dV: per (2 key blocks, sequence and KV head), over the group's heads
//           and the causal query blocks: dV = P^T dO, dK = dS^T Q, RoPE^-1
// Outputs go to the dQKV rows (token-major, ld columns) and their transpose
// (feature-major, tld tokens), as the unfused path writes them.
struct AttnBwd {
  const f16 *q, *dO;      // [B][H][Sp][hd]
  const f16 *k, *v;       // [B][KVH][Sp][hd]
  const f16 *qT, *dOT;    // per z = b*KVH + g: [hd][rep*Sp] (head r of the group at r*Sp)
  const f16* kT;          // per z: [hd][Sp]
  const float* lse;       // [B][H][Sp], from attention_prefill
  float* D;               // [B][H][Sp] scratch, written by the dQ launch
  int B, S, Sp, H, KVH, hd;
  float scale;
  f16 *dqkv, *dqkvT;
  int ld, tld, q_dim, kv_dim;
  const float4* rope;  // [hd/4][rope_ld], as EpiQKV::rope
  int rope_ld;
};
hipError_t attention_backward_fused(const AttnBwd& p, hipStream_t st);

struct AttnDecode {
  const f16* q;  // [B][H][hd]
  const f16* k;  // cache rows [s][hd] at k + b*bstride + kvh*hstride
  const f16* v;
  size_t bstride, hstride;
  const int* d_pos;  // keys 0..*d_pos are attended
  int B, H, KVH, hd, ctx_max;
  int nch;  // chunks per (sequence, head): attn_decode_chunking(ctx_max, B, H).n
  float scale;
  float* part_o;   // [B][H][nchunks][hd] unnormalised chunk outputs
  float* part_ml;  // [B][H][nchunks][2] chunk (max, sum) in log2 units
  f16* out;        // [B][H*hd], written by attention_combine, or by
                   // attention_decode itself when there is one chunk
  // Two-term fp16 inputs (common.hpp): low parts of q, k and v in the same
  // layouts, all set or all NULL; the attention rows are then split rows
  // [B][2*H*hd].
  const f16 *q_lo = nullptr, *k_lo = nullptr, *v_lo = nullptr;
  // One chunk, no low parts: out in the decode GEMV's B-fragment order over
  // K = H*hd (element (b, k) at ((k/32)*64 + b + 16*((k%32)/8))*8 + k%8, 16
  // row slots) instead of rows.
  bool out_frag = false;
};
// Chunks of the decode context for B sequences of H heads: n chunks per
// (sequence, head), each attn_chunk_keys(pos, n) keys long at position pos,
// run by workgroups of `waves` waves.
struct AttnChunking {
  int n, waves;
};
AttnChunking attn_decode_chunking(int ctx_max, int B, int H);
// Partials of the chunks that hold keys; the Wo GEMV prologue or
// attention_combine turns them into the attention output. With one chunk
// the kernel writes the attention rows (out) itself.
hipError_t attention_decode(const AttnDecode& p, hipStream_t st);
hipError_t attention_combine(const AttnDecode& p, hipStream_t st);

// ---- elementwise / reductions (elementwise.hip) ----
hipError_t embedding(const f16* E, const uint32_t* tok, int T, int dim, int vocab, float* x,
                     int* err, hipStream_t st);
// Rows r < T of x at x + r*row_stride (floats), dim contiguous; out rows are
// [T, dim], or split rows [T, 2*dim] (common.hpp).
// frag: out in the decode GEMVs' B-fragment order over 16 row slots (T <= 16;
// EpiSwiGLU::frag) instead of rows.
hipError_t rmsnorm(const float* x, long row_stride, const float* gamma, int T, int dim, float eps,
                   f16* out, float* rms_inv, hipStream_t st, bool split = false, bool frag = false);
// Per-row cross-entropy against targets (ids >= vocab: NaN loss, error bit 2).
hipError_t cross_entropy(const float* logits, const uint32_t* targets, int T, int vocab,
                         float* loss, int* err, hipStream_t st);
hipError_t mean_reduce(const float* v, int n, float* out, hipStream_t st);
hipError_t set_int(int* d, int value, hipStream_t st);

// Weight repacking: src fp32 [R][C] row-major (device), dst fp16.
//   mode 0: dst[(row0 + j) * ld + i] = src[i][j]              (transpose)
//   mode 1: dst[((j>>1)*4 + (j&1) + row0) * ld + i] = src[i][j] (W1/W3 interleave)
//   mode 2: dst[(row0 + i) * ld + j] = src[i][j]              (copy)
hipError_t repack(const float* src, int R, int C, f16* dst, int ld, int row0, int mode,
                  hipStream_t st);
// The same permutation into fp32 (the optimizer's master copy).
hipError_t repack_f32(const float* src, int R, int C, float* dst, int ld, int row0, int mode,
                      hipStream_t st);
// Elements [first, first+n) of hb_synth_normal(seed, tensor_id) as fp32.
hipError_t synth_f32(uint64_t seed, uint64_t tensor_id, float scale, uint64_t first, size_t n,
                     float* dst, hipStream_t st);
hipError_t fill_f32(float* d, float v, size_t n, hipStream_t st);
hipError_t fill_f16_zero(f16* d, size_t n, hipStream_t st);

// ---- validation windows (elementwise.hip) ----
// tok/tgt [B][S] of windows vs0 .. vs0+B-1 of a uint16 stream of n tokens
// (window w starts at (w*S) % (n - S - 1)).
hipError_t window_gather(const uint16_t* toks, uint64_t n, uint32_t vs0, int B, int S,
                         uint32_t* tok, uint32_t* tgt, hipStream_t st);
// acc[3] (fp64) += {sum loss, sum loss over byte-bearing targets, sum bytes}.
hipError_t bpb_accum(const float* loss, const uint32_t* tgt, int T, const int* tb, int tb_len,
                     double* acc, hipStream_t st);

// ---- optimizer (optimizer.hip) ----
// AdamW hyperparameters of one launch (cpu/adam.rs:95-132): omb1 = 1 - b1,
// omb2 = 1 - b2, bc1 = 1/(1 - b1^t), bc2 = 1/(1 - b2^t), all computed in fp32
// on the host; gscale is used when no device scale pointer is given.
struct AdamW {
  float lr, wd, b1, b2, omb1, omb2, eps, bc1, bc2, gscale;
};
// One fused step over n (multiple of 4) elements of param/grad/m/v; the new
// param is also written to dst16 (fp16 weights) or dst32 (fp32 gammas).
hipError_t adamw(float* p, const float* g, float* m, float* v, f16* dst16, float* dst32, size_t n,
                 const AdamW& h, const float* d_gscale, hipStream_t st);
// The same step for one matrix [R][C] that also writes its fp16 transpose
// dstT [C][ldT] (ldT >= R, multiple of 8; columns [R, ldT) zero).
hipError_t adamw_tiled(float* p, const float* g, float* m, float* v, f16* dst, f16* dstT, int R,
                       int C, int ldT, const AdamW& h, const float* d_gscale, hipStream_t st);
constexpr int SUMSQ_BLOCKS = 1024;
// partials[SUMSQ_BLOCKS] (fp64) from n per-tile fp32 sums of squares plus
// SUMSQ_BLOCKS fp64 partials of another region, in a fixed order.
hipError_t combine_sumsq(const float* slots, long n, const double* extra, double* partials,
                         hipStream_t st);
// partials[SUMSQ_BLOCKS] = fp64 sums of squares of fixed shares of g[0, n).
hipError_t grad_sumsq(const float* g, size_t n, double* partials, hipStream_t st);
struct ClipCfg {
  float gsc;        // 1 / (accum_steps * loss_scale)
  float grad_clip;  // max norm
};
// out[0] = norm, out[1] = train_step's gradient scale, out[2] = clip_grads' factor.
hipError_t grad_clip_scale(const double* partials, ClipCfg c, float* out, hipStream_t st);
hipError_t scale_inplace(float* g, size_t n, const float* d_scale, hipStream_t st);
hipError_t widen_f16(const f16* src, float* dst, size_t n, hipStream_t st);


// ---- training backward (backward.hip) ----
// dst[b][c][r] = src[b][r][c] (r < R, c < C; src rows lds apart, batches sbs /
// dbs halfs apart); dst columns [R, ldd) are zeroed.
hipError_t transpose_f16(const f16* src, int R, int C, int lds, size_t sbs, f16* dst, int ldd,
                         size_t dbs, int batch, hipStream_t st);
// dst[c][r] = fp16(scale * src[r][c]) with columns [R, ldd) zeroed; rm
// (nullable) [R][C] gets the same fp16 values row-major.
hipError_t cast_transpose(const float* src, int R, int C, float scale, f16* rm, f16* dst, int ldd,
                          hipStream_t st);
// ForwardResult's fp32 views: dlogits [T][V] = (softmax - onehot) * inv_seq
// and logits_capped [T][V] = z / softcap (each nullable).
hipError_t ce_grad_views(const float* logits, const uint32_t* tgt, int T, int V, float inv_seq,
                         float softcap, float* dl, float* tcap, hipStream_t st);
// x_prenorm / x_final (each nullable) channel-first [b][c][s] from x [B*S][d].
hipError_t final_norm_views(const float* x, const float* gamma, const float* rinv, int B, int S, int d,
                            float* pre, float* fin, hipStream_t st);
// dl [T][Vp] fp16 = (softmax(logits) - onehot) * gs (* (1 - (z/softcap)^2)).
hipError_t ce_backward(const float* logits, const uint32_t* tgt, int T, int V, int Vp, float gs,
                       float softcap, f16* dl, hipStream_t st);
// out = res + RMSNorm-backward(dy) (res nullable); dgamma += gamma gradient.
// rinv [T] and part [rmsnorm_backward_part_floats(dim)] are scratch.
// With sq (nullable), the sums of squares of the new dgamma values go to
// sq[0 .. ceil(dim / 256)).
hipError_t rmsnorm_backward(const float* dy, const float* x, const float* gamma, const float* res,
                            int T, int dim, float eps, float* out, float* rinv, float* part,
                            float* dgamma, bool accumulate, hipStream_t st, float* sq = nullptr);
size_t rmsnorm_backward_part_floats(int dim);
// dE[tok[t]] += dx[t], deterministic; tokens >= vocab are skipped.
hipError_t embedding_backward(const float* dx, const uint32_t* tok, int T, int dim, int vocab,
                              float* dE, hipStream_t st);

}  // namespace hb
