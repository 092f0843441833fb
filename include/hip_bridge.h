/*
 * hip_bridge.h — C ABI of libhip_bridge.so, the MI355X (gfx950) replacement for
 * rustane's `ane-bridge` on the transformer forward path and the single-token
 * decode loop.
 *
 * Reference boundary being replaced (paths relative to the rustane tree):
 *   crates/ane-bridge/src/lib.rs:8-9          re-export of the `ane` crate (Graph,
 *                                             Executable, TensorData) that every
 *                                             forward kernel is built and run through
 *   crates/engine/src/layer.rs:239-274        CompiledKernels::compile (graph build)
 *   crates/engine/src/layer.rs:684-806        per-layer dispatch (run_cached_direct)
 *   crates/engine/src/full_model.rs:187-247   forward_ws (model forward + mean loss)
 *   crates/engine/src/full_model.rs:717-767   forward_losses (per-position losses)
 *   crates/metal-decode/src/lib.rs:1-8        planned single-token decode (placeholder)
 * and, for training, the rows next to that path:
 *   crates/engine/src/full_model.rs:250-331   backward_ws (with layer.rs:1606-1858)
 *   crates/engine/src/full_model.rs:487-714   update_weights / grad_norm / train_step
 *   crates/engine/src/bin/train.rs:123-202    validation loop, RSTK checkpoints
 *
 * Conventions
 *   - Every entry point returns int: 0 (HB_OK) on success, a negative HB_E_* code
 *     on failure. hb_last_error() returns a thread-local message for the last
 *     failure on the calling thread. Nothing throws across the ABI.
 *   - Host pointers ("h_" in the docs) are borrowed for the duration of the call.
 *     Device pointers ("d_") must point to memory on the context's device.
 *   - Entry points taking host buffers are synchronous. Entry points documented
 *     as "async" enqueue on the context stream and return immediately.
 *   - A context is single-owner, as the reference's CompiledKernels/IOSurfaces
 *     are: use one context per host thread.
 *   - Weights are passed in the reference's fp32 layouts (layer.rs:16-26,
 *     full_model.rs:13-17) and are converted to fp16 and repacked on the device.
 *   - Token ids are uint32 as in the reference (full_model.rs:191-192).
 */
#ifndef HIP_BRIDGE_H
#define HIP_BRIDGE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes --------------------------------------------------------- */
enum {
  HB_OK = 0,
  HB_E_INVALID = -1, /* bad argument: null pointer, out-of-range size or token */
  HB_E_CONFIG = -2,  /* model config rejected (see hb_model_create)            */
  HB_E_DEVICE = -3,  /* HIP runtime error (launch, copy, sync)                 */
  HB_E_OOM = -4,     /* device allocation failed                               */
  HB_E_STATE = -5,   /* call out of order (e.g. weights not uploaded, KV full) */
  HB_E_INJECTED = -6 /* error injected by hb_debug_inject_error                */
};

/* ---- dtypes --------------------------------------------------------------- */
enum { HB_DTYPE_F16 = 1 };

typedef struct hb_ctx hb_ctx;
typedef struct hb_model hb_model;
typedef struct hb_kv hb_kv;
typedef struct hb_opt hb_opt;
typedef struct hb_tokens hb_tokens;

/*
 * Model shape. Field names and meaning follow rustane's ModelConfig
 * (crates/engine/src/model.rs:5-17); the last four fields are the constants the
 * reference hard-codes: RoPE base 10000 (kernels/sdpa_fwd.rs:22), RMSNorm eps
 * 1e-5 (cpu/rmsnorm.rs:10), residual scale 1/sqrt(2*nlayers) (layer.rs:698,
 * kernels/ffn_fused.rs:29) and logit softcap (full_model.rs:234-239, default 0).
 * `seq` is the longest sequence hb_forward accepts. q_dim must equal heads*hd and
 * kv_dim kv_heads*hd; gqa_ratio = heads/kv_heads.
 */
typedef struct hb_model_config {
  int32_t dim;
  int32_t hidden;
  int32_t heads;
  int32_t kv_heads;
  int32_t hd;
  int32_t seq;
  int32_t nlayers;
  int32_t vocab;
  int32_t q_dim;
  int32_t kv_dim;
  int32_t gqa_ratio;
  float rope_theta;     /* 0 -> 10000                 */
  float norm_eps;       /* 0 -> 1e-5                  */
  float residual_alpha; /* 0 -> 1/sqrt(2*nlayers)     */
  float softcap;        /* 0 -> no softcap            */
} hb_model_config;

/* ---- library / context ---------------------------------------------------- */

/* "hip-gfx950". Replaces nothing in the reference (the ANE backend is implicit). */
const char* hb_backend_name(void);
/* Message for the last failing call on this thread ("" if none). */
const char* hb_last_error(void);
/* Number of visible HIP devices (0 on a host without a GPU). */
int hb_device_count(int* out_count);

/* Create a context on `device`: owns a HIP stream (default priority). */
int hb_ctx_create(int device, hb_ctx** out);
int hb_ctx_destroy(hb_ctx* ctx);
/* Use a caller-owned hipStream_t for all work of this context (NULL restores
 * the context's own stream). The stream must belong to the context's device. */
int hb_ctx_set_stream(hb_ctx* ctx, void* hip_stream);
int hb_ctx_get_stream(hb_ctx* ctx, void** hip_stream);
/* Wait for all work on the context stream; reports device-side input errors
 * (an out-of-range token seen by an async entry point) as HB_E_INVALID. */
int hb_ctx_synchronize(hb_ctx* ctx);

/* ---- model ---------------------------------------------------------------- */

/*
 * Validate `cfg` and allocate the device model (weights only; activations are
 * sized on first use). Replaces CompiledKernels::compile (layer.rs:239-274).
 * Requirements (HB_E_CONFIG otherwise): all dims > 0; dim, hidden, q_dim,
 * kv_dim and vocab multiples of 64; hd in {64, 128}; q_dim == heads*hd;
 * kv_dim == kv_heads*hd; heads % kv_heads == 0; dtype == HB_DTYPE_F16.
 */
int hb_model_create(hb_ctx* ctx, const hb_model_config* cfg, int dtype, hb_model** out);
/* The same validation without a device: fills the defaulted fields of *cfg in
 * place and returns HB_OK or HB_E_CONFIG. */
int hb_config_validate(hb_model_config* cfg);
int hb_model_destroy(hb_model* model);
/* The effective config (defaults filled in). */
int hb_model_get_config(const hb_model* model, hb_model_config* out);
/* Bytes of device memory held by weights. */
int hb_model_weight_bytes(const hb_model* model, uint64_t* out);
/* Logit softcap for later forwards (0 = off). The reference passes it per call
 * (forward_ws(..., softcap, ..), full_model.rs:187-195). */
int hb_model_set_softcap(hb_model* model, float softcap);
/*
 * Precision of the first layers (no counterpart in the reference, whose ANE
 * graphs compute in fp16 throughout). The first n layers of later forwards
 * (hb_forward*, hb_prefill, and the decode steps of KV caches created after
 * the call) feed their products two-term fp16 operands, hi + lo with
 * lo = fp16(x - fp16(x)): GEMM/GEMV inputs, Q, K, V and attention
 * probabilities carry ~22 significant bits instead of 11, at twice the MFMA
 * work of those layers (the weights are still read once). Rounding inside the
 * first layer, where the residual stream is still the small embedding, sets
 * most of a deep model's distance from fp32 arithmetic. Default 1; 0 <= n <=
 * nlayers; with n = nlayers the final norm's rows feeding the logits are
 * split too (fp32 arithmetic on the fp16 weights, to accumulation order). The
 * training entry points and hb_op_* are not affected.
 */
int hb_model_set_precise_layers(hb_model* model, int n);
int hb_model_get_precise_layers(const hb_model* model, int* out_n);

/*
 * Upload one layer's weights from host fp32 arrays in the reference layouts
 * (LayerWeights, layer.rs:16-26):
 *   wq [dim*q_dim], wk [dim*kv_dim], wv [dim*kv_dim]   element [c*out + j]
 *   wo [q_dim*dim]                                      element [j*dim + c]
 *   w1, w3 [dim*hidden]                                 element [c*hidden + k]
 *   w2 [dim*hidden] (used transposed, ffn_fused.rs:65-72) element [c*hidden + k]
 *   gamma1, gamma2 [dim]
 */
int hb_model_upload_layer(hb_model* model, int layer, const float* wq, const float* wk,
                          const float* wv, const float* wo, const float* w1, const float* w3,
                          const float* w2, const float* gamma1, const float* gamma2);
/* Tied embedding E [vocab*dim] (element [v*dim + c]) and final gamma [dim]
 * (ModelWeights, full_model.rs:13-17). */
int hb_model_upload_embed(hb_model* model, const float* embed, const float* gamma_final);
/*
 * Fill every weight on the device with the seeded synthetic values that
 * hb_synth_normal produces on the host for the same (seed, tensor id), with
 * gammas = 1 — bit-identical to uploading those host arrays. Tensor ids:
 * layer l: wq 16l+0, wk 16l+1, wv 16l+2, wo 16l+3, w1 16l+4, w3 16l+5,
 * w2 16l+6; embedding: HB_SYNTH_EMBED_ID.
 */
int hb_model_init_synthetic(hb_model* model, uint64_t seed, float std);

/* ---- seeded synthetic inputs (host, deterministic) ------------------------- */
#define HB_SYNTH_EMBED_ID 0xFFFFu
/* out[i], i < n: approximately N(0, std^2) (standardised sum of eight uniform
 * 16-bit draws of a counter-based hash of (seed, tensor_id, i)). */
int hb_synth_normal(uint64_t seed, uint64_t tensor_id, float std, uint64_t n, float* out);
/* out[i], i < n: uniform over [0, vocab) from the same hash. */
int hb_synth_tokens(uint64_t seed, uint64_t stream, uint32_t vocab, uint64_t n, uint32_t* out);

/* ---- forward (prefill) ----------------------------------------------------- */

/*
 * Full forward over B independent sequences of S tokens (token-major
 * [B*S]): embedding -> nlayers x layer -> final RMSNorm -> tied logits ->
 * optional softcap -> cross-entropy. Mirrors forward_ws / forward_losses
 * (full_model.rs:187-247, 717-767); B > 1 is B independent B=1 calls.
 * Synchronous. targets may be NULL (no loss); per_pos_loss [B*S], logits
 * [B*S*vocab] and mean_loss (mean over all B*S positions) may each be NULL.
 * Requires 1 <= S <= cfg.seq.
 */
int hb_forward(hb_model* model, const uint32_t* h_tokens, const uint32_t* h_targets, int B,
               int S, float* h_per_pos_loss, float* h_logits, float* h_mean_loss);
/* Same on device buffers; async on the context stream. Out-of-range tokens
 * are not read (the row is zeroed) and make the next hb_ctx_synchronize fail. */
int hb_forward_device(hb_model* model, const uint32_t* d_tokens, const uint32_t* d_targets,
                      int B, int S, float* d_per_pos_loss, float* d_logits, float* d_mean_loss);
/* Pre-size activation buffers for forwards of up to B sequences of S tokens
 * so that later calls of that size allocate nothing. */
int hb_model_reserve(hb_model* model, int B, int S);

/*
 * Device time of each stage of one forward. Replaces ForwardTimings /
 * forward_timed (layer.rs:821-1015), which time one layer's CPU norms, the
 * staging of each ANE input, the three ANE graphs and the readbacks; here the
 * inputs stay on the device (no staging or readback stage) and each stage is
 * the kernels between two HIP events on the stream:
 *   rmsnorm1_ms           the separate input norms (layer 0's; later layers'
 *                         come out of the previous W2 reduction, below)
 *   sdpa_qkv_ms           Q/K/V projection + RoPE + K/V^T scatter   (sdpaFwd)
 *   sdpa_attention_ms     causal attention                          (sdpaFwd)
 *   wo_ms                 Wo projection (split-K partial sums)      (woFwd)
 *   residual_rmsnorm2_ms  split-K reduction + residual + RMSNorm2
 *   ffn_up_ms             W1|W3 projection + SwiGLU                 (ffnFused)
 *   ffn_down_ms           W2 projection (split-K partial sums)      (ffnFused)
 *   ffn_residual_norm_ms  its reduction + residual + the next layer's norm
 * The per-layer stages are summed over layers 1 .. nlayers-1
 * (layers_summed of them); the first layer, on two-term operands by default
 * (hb_model_set_precise_layers), is layer0_ms. total_ms spans the whole
 * forward, embedding to mean loss. The events add a little time of their
 * own between launches.
 */
typedef struct hb_forward_timings {
  float embedding_ms;
  float rmsnorm1_ms;
  float sdpa_qkv_ms;
  float sdpa_attention_ms;
  float wo_ms;
  float residual_rmsnorm2_ms;
  float ffn_up_ms;
  float ffn_down_ms;
  float ffn_residual_norm_ms;
  float logits_ms;
  float cross_entropy_ms;
  float layer0_ms;
  float total_ms;
  int32_t layers_summed;
} hb_forward_timings;
/* hb_forward_device's launches run eagerly with an event after each stage;
 * synchronous. Losses and mean (nullable device buffers) equal
 * hb_forward_device's bit for bit. */
int hb_forward_timed(hb_model* model, const uint32_t* d_tokens, const uint32_t* d_targets, int B, int S,
                     float* d_per_pos_loss, float* d_mean_loss, hb_forward_timings* out);

/* ---- per-kernel entry points (device buffers, async) -----------------------
 * The reference runs each layer as CPU RMSNorm -> sdpaFwd -> woFwd -> CPU
 * residual + RMSNorm -> ffnFused (layer.rs:684-806). These expose the same
 * split so each stage can be checked on its own. T = B*S token rows. */

/* RMSNorm over rows of x [T, dim] fp32 -> out fp16 [T, dim]; rms_inv [T] fp32
 * (nullable). cpu/rmsnorm.rs:149-183. */
int hb_op_rmsnorm(hb_ctx* ctx, const float* d_x, const float* d_gamma, int T, int dim, float eps,
                  void* d_out_f16, float* d_rms_inv);
/* x[t, :] = E[tokens[t], :] as fp32 (cpu/embedding.rs:8-16). */
int hb_op_embedding(hb_model* model, const uint32_t* d_tokens, int T, float* d_x);
/*
 * sdpaFwd (kernels/sdpa_fwd.rs:49-161): Q/K/V projections of xnorm (fp16
 * [B*S, dim]), interleaved RoPE on Q and K, causal softmax attention. Writes
 * attn_out fp16 [B*S, q_dim] (channel h*hd+e). If d_qkv_tap is non-NULL it also
 * receives fp32 [B*S, q_dim + 2*kv_dim] = Q_rope | K_rope | V.
 */
int hb_op_sdpa_fwd(hb_model* model, int layer, const void* d_xnorm_f16, int B, int S,
                   void* d_attn_f16, float* d_qkv_tap);
/* woFwd + residual (dyn_matmul.rs:15-46, layer.rs:784):
 * x2 = x + alpha * attn @ Wo, x and x2 fp32 [T, dim]. */
int hb_op_wo_fwd(hb_model* model, int layer, const void* d_attn_f16, const float* d_x, int T,
                 float* d_x2);
/* hb_op_wo_fwd without any allocation. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The split-K
 * partial sums live in a fixed 16 MiB device array inside the library (one per
 * GPU, held until the process ends), which covers every shape; results equal
 * hb_op_wo_fwd's bit for bit. Calls on one GPU share that array: outside a
 * graph capture each call waits (on its stream) for the previous call's use
 * of it, so calls from different streams or contexts run one after another;
 * under capture no such wait is recorded, and graph replays that overlap on
 * one GPU race -- keep them ordered on one stream. */
int hb_op_wo_fwd_noalloc(hb_model* model, int layer, const void* d_attn_f16, const float* d_x, int T,
                         float* d_x2);
/*
 * ffnFused (kernels/ffn_fused.rs:22-83): h1 = xn@W1, h3 = xn@W3,
 * gate = silu(h1)*h3, x_next = x2 + alpha * gate @ W2^T. xn fp16 [T, dim], x2
 * and x_next fp32 [T, dim]. Taps (nullable): h13 fp32 [T, 2*hidden] = h1 | h3,
 * gate fp16 [T, hidden].
 */
int hb_op_ffn_fused(hb_model* model, int layer, const void* d_x2norm_f16, const float* d_x2,
                    int T, float* d_x_next, float* d_h13_tap, void* d_gate_f16);
/* The up half of ffnFused alone (one kernel: W1|W3 GEMM with the SwiGLU gate
 * formed in its epilogue): gate fp16 [T, hidden] = silu(xn@W1) * (xn@W3). */
int hb_op_ffn_up(hb_model* model, int layer, const void* d_x2norm_f16, int T, void* d_gate_f16,
                 float* d_h13_tap);
/* Final stage (full_model.rs:228-246): logits = xf @ E^T (+softcap), then
 * per-row cross-entropy (cpu/cross_entropy.rs:58-96) when targets != NULL.
 * xf fp16 [T, dim]; logits fp32 [T, vocab] (nullable only if losses wanted);
 * losses fp32 [T] (nullable). */
int hb_op_logits_ce(hb_model* model, const void* d_xf_f16, const uint32_t* d_targets, int T,
                    float* d_logits, float* d_losses);
/* Plain C[M,N] = A[M,K] @ B[N,K]^T, fp16 inputs, fp32 output, on the same
 * MFMA kernel the model GEMMs use. K % 64 == 0, N % 4 == 0. */
int hb_op_gemm_nt(hb_ctx* ctx, const void* d_a_f16, const void* d_b_f16, float* d_c, int M,
                  int N, int K);

/* ---- single-token decode (the loop metal-decode/src/lib.rs:1-8 plans) ----- */

/* Preallocate a contiguous fp16 KV cache for `batch` sequences of up to
 * ctx_max positions: [nlayers][batch][K,V][kv_heads][ctx_max][hd]. */
int hb_kv_create(hb_model* model, int batch, int ctx_max, hb_kv** out);
int hb_kv_destroy(hb_kv* kv);
/* Forget all positions (length -> 0). */
int hb_kv_reset(hb_kv* kv);
int hb_kv_length(hb_kv* kv, int* out_len);
/* Bytes of device memory held by the cache. */
int hb_kv_bytes(hb_kv* kv, uint64_t* out);
/*
 * Run the prompt tokens [batch*S] (token-major per sequence) through the
 * forward path, writing K/V for positions [0, S) into the cache. Returns the
 * last position's logits [batch*vocab] and greedy next token [batch]
 * (nullable). Requires an empty cache and S <= ctx_max.
 */
int hb_prefill(hb_model* model, hb_kv* kv, const uint32_t* h_tokens, int S, float* h_logits,
               uint32_t* h_next);
/*
 * One decode step: tokens [batch] at position p = current length; appends
 * K/V at p, returns logits [batch*vocab] and argmax [batch] (nullable), and
 * advances the length. Logits at p equal row p of a full forward over the
 * same token history.
 */
int hb_decode_step(hb_model* model, hb_kv* kv, const uint32_t* h_tokens, float* h_logits,
                   uint32_t* h_next);
/*
 * nsteps greedy steps entirely on the device: each step consumes the previous
 * step's argmax (the first consumes h_first [batch]); writes the generated
 * tokens [nsteps*batch] to h_out (nullable). The step is replayed from one
 * captured HIP graph.
 */
int hb_decode_greedy(hb_model* model, hb_kv* kv, const uint32_t* h_first, int nsteps,
                     uint32_t* h_out);

/* ---- optimizer: fused AdamW, gradient norm and clipping -------------------- */

/* TrainConfig (full_model.rs:33-70): the fields the optimizer step reads. */
typedef struct hb_train_config {
  float max_lr;          /* 3e-4   */
  float min_lr_frac;     /* 0.1    */
  uint32_t warmup_steps; /* 100    */
  uint32_t total_steps;  /* 10000  */
  float beta1;           /* 0.9    */
  float beta2;           /* 0.95   */
  float eps;             /* 1e-8   */
  float weight_decay;    /* 0.1    */
  float matrix_lr_scale; /* 0.05   */
  float embed_lr_scale;  /* 5.0    */
  float loss_scale;      /* 256    */
  uint32_t accum_steps;  /* 10     */
  float grad_clip;       /* 1.0    */
} hb_train_config;

/* learning_rate (full_model.rs:334-342): linear warmup, then cosine decay to
 * max_lr * min_lr_frac, in fp32 as the reference computes it. */
int hb_learning_rate(const hb_train_config* tc, uint32_t step, float* out_lr);

/*
 * Optimizer state of a model: ModelOptState (full_model.rs:26-31) plus the
 * ModelGrads arena (full_model.rs:20-24) and an fp32 master copy of every
 * weight, all on the device in the packed order of the fp16 weights (one
 * fused pass updates master, m, v and the fp16 copy; 4 fp32 arenas, 16 bytes
 * per parameter). m, v and the gradients start at 0; the master copy starts
 * from the model's current fp16 weights, or from fp32 values given by
 * hb_opt_upload_layer / hb_opt_upload_embed / hb_opt_init_synthetic.
 */
int hb_opt_create(hb_model* model, const hb_train_config* tc, hb_opt** out);
int hb_opt_destroy(hb_opt* opt);
/* fp32 weights in the reference layouts of hb_model_upload_layer/_embed
 * (layer.rs:16-26, full_model.rs:13-17): written to the master copy and, as
 * fp16, to the model. */
int hb_opt_upload_layer(hb_opt* opt, int layer, const float* wq, const float* wk, const float* wv,
                        const float* wo, const float* w1, const float* w3, const float* w2,
                        const float* gamma1, const float* gamma2);
int hb_opt_upload_embed(hb_opt* opt, const float* embed, const float* gamma_final);
/* hb_model_init_synthetic into the master copy and the model. */
int hb_opt_init_synthetic(hb_opt* opt, uint64_t seed, float std);
/* Gradients in the reference layouts (LayerGrads, layer.rs:29-39: dwq [dim*q],
 * ..., dw2 [dim*hidden], dgamma1, dgamma2; dembed, dgamma_final), replacing
 * the arena's contents for that layer / the embedding. */
int hb_opt_upload_grads_layer(hb_opt* opt, int layer, const float* dwq, const float* dwk,
                              const float* dwv, const float* dwo, const float* dw1,
                              const float* dw3, const float* dw2, const float* dgamma1,
                              const float* dgamma2);
int hb_opt_upload_grads_embed(hb_opt* opt, const float* dembed, const float* dgamma_final);
/* ModelGrads::zero_out (train_step, full_model.rs:670). Until the arena's
 * pointer has been handed out (hb_opt_grad_arena) the clearing is deferred:
 * every hb_opt_* call that reads or partly writes the gradients clears them
 * first, and hb_forward_backward stores every element instead (the 27 GB
 * fill of a 7B arena is then never done). */
int hb_opt_zero_grads(hb_opt* opt);
/* The device gradient arena (fp32, packed order) for producers on the device:
 * pointer and length in floats. After this call the library no longer
 * assumes a zeroed arena stays untouched, so hb_forward_backward always adds
 * (it otherwise stores onto an arena that hb_opt_zero_grads just cleared:
 * the same values with half the gradient traffic). */
int hb_opt_grad_arena(hb_opt* opt, float** d_grads, uint64_t* n_floats);
/* grad_norm (full_model.rs:600-622): global L2 norm of all gradients. */
int hb_opt_grad_norm(hb_opt* opt, float* out_norm);
/* clip_grads (full_model.rs:625-641): scale all gradients by max_norm/norm
 * when norm > max_norm. The norm (nullable) is returned. */
int hb_opt_clip_grads(hb_opt* opt, float max_norm, float* out_norm);
/* update_weights (full_model.rs:487-592) with step count t (1-based) and base
 * learning rate lr: matrices at lr*matrix_lr_scale with weight decay, the
 * embedding at lr*embed_lr_scale and the gammas at lr without; gradients
 * multiplied by grad_scale inline. Asynchronous on the context stream. */
int hb_opt_update_weights(hb_opt* opt, uint32_t t, float lr, float grad_scale);
/* The optimizer half of train_step (full_model.rs:697-711) after `step`
 * completed microbatches of accumulation: grad norm, the combined
 * descale/clip factor (decided on the device: no host round trip),
 * learning_rate(step), update_weights(t = step + 1). out_norm (nullable)
 * receives the raw norm, which waits for the step to finish. */
int hb_opt_step(hb_opt* opt, uint32_t step, float* out_norm);
/* (After hb_forward_backward the norm of hb_opt_step / hb_opt_grad_norm is
 * assembled from sums of squares the backward took while writing the
 * gradients -- no second pass over the arena -- until anything else writes
 * the gradients.) */
/* Read state back in the reference layouts: which = 0 master weights, 1 m,
 * 2 v, 3 gradients. */
int hb_opt_download_layer(hb_opt* opt, int layer, int which, float* wq, float* wk, float* wv,
                          float* wo, float* w1, float* w3, float* w2, float* gamma1,
                          float* gamma2);
int hb_opt_download_embed(hb_opt* opt, int which, float* embed, float* gamma_final);

/* ---- training forward + backward ------------------------------------------ */

/* forward_ws + backward_ws (full_model.rs:187-247 and 250-331, the per-layer
 * backward of layer.rs:1606-1858) on B sequences of S tokens: the forward
 * keeps every layer's activations, the backward ADDS the gradients of
 * loss_scale * (mean cross-entropy of each sequence) to opt's fp32 gradient
 * arena (the reference accumulates into ModelGrads the same way; train_step
 * divides loss_scale and the accumulation count back out, hb_opt_step).
 * Softcap comes from the model config. Per-position losses (nullable, [B*S])
 * and their mean (nullable) are returned. Host ids, synchronous; opt must
 * belong to m. The first call allocates fp16 transposed weight copies (the
 * size of the weights) and the activations for (B, S). */
int hb_forward_backward(hb_model* m, hb_opt* opt, const uint32_t* tokens,
                        const uint32_t* targets, int B, int S, float loss_scale,
                        float* per_pos_loss, float* mean_loss);
/* The same with ids in device memory; asynchronous on the context stream,
 * losses written to device pointers (nullable). Ids >= vocab are reported
 * through the context's error word by the forward and skipped by the
 * embedding backward. */
int hb_forward_backward_device(hb_model* m, hb_opt* opt, const uint32_t* d_tokens,
                               const uint32_t* d_targets, int B, int S, float loss_scale,
                               float* d_loss, float* d_mean);

/* The reference's forward/backward pair, split across two calls.
 *
 * ForwardResult (full_model.rs:73-81): host views that forward() returns
 * besides the loss and the per-layer caches, each nullable, B sequences one
 * after another in the reference's per-sequence layouts:
 *   dlogits       [B*S*vocab]  (softmax - onehot(target)) / S, the gradient
 *                              of the sequence's mean CE (cross_entropy.rs:58-96)
 *   x_final       [B][dim][S]  channel-first, after the final RMSNorm
 *   x_prenorm     [B][dim][S]  channel-first, before it
 *   rms_inv_final [B*S]
 *   logits_capped [B*S*vocab]  tanh(logits / softcap), written only when the
 *                              model's softcap is > 0 (the reference leaves it
 *                              empty otherwise) */
typedef struct hb_forward_result {
  float* dlogits;
  float* x_final;
  float* x_prenorm;
  float* rms_inv_final;
  float* logits_capped;
} hb_forward_result;

/* forward (full_model.rs:345-410) for training: the forward of
 * hb_forward_backward on B sequences of S tokens (host ids, synchronous),
 * keeping every layer's activations on the device -- ForwardResult.caches --
 * for the next hb_train_backward on this model. Per-position losses
 * (nullable, [B*S]), their mean (nullable) and the views in *out (nullable)
 * are returned. Any other training call on the model drops the kept caches. */
int hb_train_forward(hb_model* m, const uint32_t* h_tokens, const uint32_t* h_targets, int B, int S,
                     float* h_per_pos_loss, float* h_mean_loss, const hb_forward_result* out);
/* backward (full_model.rs:414-483) from the caches of the last
 * hb_train_forward: ADDS the gradients of loss_scale * (mean CE of each
 * sequence) to opt's gradient arena, as hb_forward_backward does. The
 * softcap is the one the kept forward ran with (the reference passes the
 * forward's softcap again), even if hb_model_set_softcap or an inference
 * forward changed the model's since. HB_E_STATE without a kept forward
 * (each forward serves one backward). Synchronous. */
int hb_train_backward(hb_model* m, hb_opt* opt, float loss_scale);

/* ---- RSTK checkpoints (bin/train.rs:165-202) ------------------------------ */

/* Header of the reference's checkpoint file: "RSTK", then little-endian u32
 * version (1), step, dim, nlayers, vocab, seq (28 bytes), followed by fp32
 * weights in the order embed, gamma_final, then per layer wq, wk, wv, wo, w1,
 * w3, w2, gamma1, gamma2 in the reference layouts. */
typedef struct hb_rstk_header {
  uint32_t version, step, dim, nlayers, vocab, seq;
} hb_rstk_header;

/* Read and check a checkpoint's header (host only, no device): HB_E_INVALID
 * for a missing file, a bad magic or version. */
int hb_rstk_read_header(const char* path, hb_rstk_header* out);
/* Load a checkpoint into the model -- as hb_model_upload_layer/_embed, and
 * into the optimizer's fp32 master copy when opt != NULL. The header's dim,
 * nlayers and vocab must match the model (HB_E_CONFIG) and the file size must
 * be exactly what the model's shapes give (HB_E_INVALID); the checkpoint's seq
 * is informational. out_step (nullable) receives the header's step.
 * The reference writes these files but has no loader. */
int hb_model_load_rstk(hb_model* model, hb_opt* opt, const char* path, uint32_t* out_step);
/* Write a checkpoint with save_checkpoint's byte layout (bin/train.rs:165-202):
 * from the optimizer's fp32 master weights when opt != NULL, else from the
 * model's fp16 weights widened to fp32. */
int hb_model_save_rstk(hb_model* model, hb_opt* opt, uint32_t step, const char* path);

/* ---- data path and validation (data.rs, bin/train.rs:123-163) ------------- */

/* A token stream -- TokenData (data.rs:11-40): flat little-endian uint16 ids,
 * as the train/val .bin files hold them -- copied to the device once. */
int hb_tokens_create(hb_ctx* ctx, const uint16_t* h_tokens, uint64_t n, hb_tokens** out);
/* TokenData::open: map the file and copy it to the device (HB_E_INVALID for a
 * missing file or an odd byte count). */
int hb_tokens_open(hb_ctx* ctx, const char* path, hb_tokens** out);
int hb_tokens_destroy(hb_tokens* t);
int hb_tokens_length(const hb_tokens* t, uint64_t* out_n);
/*
 * validate (bin/train.rs:123-163) on the device: window vs (0 <= vs < steps)
 * starts at pos = (vs * seq) % (n - seq - 1) with seq = the model's seq;
 * each window's per-position losses (forward_losses, full_model.rs:717-767)
 * are summed on the device, and with token_bytes [tb_len] (TokenBytes,
 * data.rs:43-58; nullable) so are the losses and byte lengths of targets with
 * a positive byte count (compute_bpb, data.rs:61-83). `batch` windows run per
 * forward (1 = the reference's one window per call; larger batches give the
 * same windows through the batched GEMMs, so the sums agree to rounding).
 * Outputs (each nullable): mean loss per token, val_bpb = nats / (ln 2 *
 * bytes), and the totals. Synchronous; HB_E_INVALID if the stream holds an id
 * outside the vocabulary or fewer than seq + 2 tokens.
 */
int hb_validate(hb_model* model, const hb_tokens* val, const int32_t* token_bytes, int tb_len,
                int steps, int batch, float* out_avg_loss, float* out_bpb, double* out_nats,
                uint64_t* out_bytes);

/* ---- failure injection (host-side test hook) ------------------------------ */
/* While `code` != 0, every entry point above except hb_last_error,
 * hb_backend_name and this one returns HB_E_INJECTED without touching the GPU. */
int hb_debug_inject_error(int code);

#ifdef __cplusplus
}
#endif
#endif /* HIP_BRIDGE_H */
