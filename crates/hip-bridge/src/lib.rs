//! hip-bridge: Rust bindings to `libhip_bridge.so`, the MI355X (gfx950) HIP
//! library behind `include/hip_bridge.h`.
//!
//! It replaces `crates/ane-bridge` (whose `src/lib.rs:8-9` re-exports the
//! `ane` crate: `Graph`, `Executable`, `TensorData`), which the engine builds
//! and runs every forward kernel through (`layer.rs:239-274` compile,
//! `layer.rs:684-806` dispatch). Here the kernels live behind a C ABI and the
//! engine keeps its model-level API: `ModelConfig` (`model.rs:5-17`),
//! `CompiledKernels::compile`, `forward_ws` / `forward` / `forward_losses`
//! (`full_model.rs:187-247, 345-410, 717-767`), `backward`
//! (`full_model.rs:414-483`) and the decode loop `metal-decode` plans.
//!
//! [`sys`] declares every entry point of the header one for one (a CPU test in
//! the repository checks names, argument counts, argument types and constness
//! against `include/hip_bridge.h`). The rest of this file is a thin safe layer:
//! owned handles that free themselves, slices checked against the model's
//! shapes, and `Result<_, HbError>` instead of status codes. Status codes map
//! to `HbError { code, message }` with the library's thread-local message; the
//! reference turns ANE failures into panics (`.expect("ANE eval failed")`,
//! `layer.rs:727`), callers that want that keep doing `.expect(..)`.
//!
//! Threading follows the library: a `Context` (one HIP stream) and everything
//! created from it belong to one host thread at a time, like the reference's
//! single-owner `CompiledKernels`. The handles are `Send` but not `Sync`.
#![allow(non_camel_case_types)]

use std::ffi::{c_int, CStr, CString};
use std::marker::PhantomData;
use std::path::Path;
use std::ptr;

/// Raw declarations of `include/hip_bridge.h`.
pub mod sys {
    use std::ffi::{c_char, c_int, c_void};

    pub const HB_OK: c_int = 0;
    pub const HB_E_INVALID: c_int = -1;
    pub const HB_E_CONFIG: c_int = -2;
    pub const HB_E_DEVICE: c_int = -3;
    pub const HB_E_OOM: c_int = -4;
    pub const HB_E_STATE: c_int = -5;
    pub const HB_E_INJECTED: c_int = -6;
    pub const HB_DTYPE_F16: c_int = 1;
    pub const HB_SYNTH_EMBED_ID: u64 = 0xFFFF;

    #[repr(C)]
    pub struct hb_ctx {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct hb_model {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct hb_kv {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct hb_opt {
        _private: [u8; 0],
    }
    #[repr(C)]
    pub struct hb_tokens {
        _private: [u8; 0],
    }

    /// ModelConfig (model.rs:5-17) plus RoPE base, RMSNorm eps, residual
    /// scale and softcap; zero selects the reference's constant.
    #[repr(C)]
    #[derive(Debug, Clone, Copy, Default, PartialEq)]
    pub struct hb_model_config {
        pub dim: i32,
        pub hidden: i32,
        pub heads: i32,
        pub kv_heads: i32,
        pub hd: i32,
        pub seq: i32,
        pub nlayers: i32,
        pub vocab: i32,
        pub q_dim: i32,
        pub kv_dim: i32,
        pub gqa_ratio: i32,
        pub rope_theta: f32,
        pub norm_eps: f32,
        pub residual_alpha: f32,
        pub softcap: f32,
    }

    /// TrainConfig (full_model.rs:33-70), the fields the optimizer reads.
    #[repr(C)]
    #[derive(Debug, Clone, Copy, Default, PartialEq)]
    pub struct hb_train_config {
        pub max_lr: f32,
        pub min_lr_frac: f32,
        pub warmup_steps: u32,
        pub total_steps: u32,
        pub beta1: f32,
        pub beta2: f32,
        pub eps: f32,
        pub weight_decay: f32,
        pub matrix_lr_scale: f32,
        pub embed_lr_scale: f32,
        pub loss_scale: f32,
        pub accum_steps: u32,
        pub grad_clip: f32,
    }

    /// Per-stage device time of one forward (ForwardTimings, layer.rs:821-1015):
    /// stage sums over layers 1..nlayers-1, the first layer in layer0_ms.
    #[repr(C)]
    #[derive(Debug, Clone, Copy, Default, PartialEq)]
    pub struct hb_forward_timings {
        pub embedding_ms: f32,
        pub rmsnorm1_ms: f32,
        pub sdpa_qkv_ms: f32,
        pub sdpa_attention_ms: f32,
        pub wo_ms: f32,
        pub residual_rmsnorm2_ms: f32,
        pub ffn_up_ms: f32,
        pub ffn_down_ms: f32,
        pub ffn_residual_norm_ms: f32,
        pub logits_ms: f32,
        pub cross_entropy_ms: f32,
        pub layer0_ms: f32,
        pub total_ms: f32,
        pub layers_summed: i32,
    }

    /// ForwardResult's host views (full_model.rs:73-81); each pointer nullable.
    #[repr(C)]
    #[derive(Debug, Clone, Copy)]
    pub struct hb_forward_result {
        pub dlogits: *mut f32,
        pub x_final: *mut f32,
        pub x_prenorm: *mut f32,
        pub rms_inv_final: *mut f32,
        pub logits_capped: *mut f32,
    }

    /// RSTK checkpoint header after the magic (bin/train.rs:165-202).
    #[repr(C)]
    #[derive(Debug, Clone, Copy, Default, PartialEq, Eq)]
    pub struct hb_rstk_header {
        pub version: u32,
        pub step: u32,
        pub dim: u32,
        pub nlayers: u32,
        pub vocab: u32,
        pub seq: u32,
    }

    extern "C" {
        // library / context
        pub fn hb_backend_name() -> *const c_char;
        pub fn hb_last_error() -> *const c_char;
        pub fn hb_device_count(out_count: *mut c_int) -> c_int;
        pub fn hb_ctx_create(device: c_int, out: *mut *mut hb_ctx) -> c_int;
        pub fn hb_ctx_destroy(ctx: *mut hb_ctx) -> c_int;
        pub fn hb_ctx_set_stream(ctx: *mut hb_ctx, hip_stream: *mut c_void) -> c_int;
        pub fn hb_ctx_get_stream(ctx: *mut hb_ctx, hip_stream: *mut *mut c_void) -> c_int;
        pub fn hb_ctx_synchronize(ctx: *mut hb_ctx) -> c_int;

        // model
        pub fn hb_model_create(
            ctx: *mut hb_ctx,
            cfg: *const hb_model_config,
            dtype: c_int,
            out: *mut *mut hb_model,
        ) -> c_int;
        pub fn hb_config_validate(cfg: *mut hb_model_config) -> c_int;
        pub fn hb_model_destroy(model: *mut hb_model) -> c_int;
        pub fn hb_model_get_config(model: *const hb_model, out: *mut hb_model_config) -> c_int;
        pub fn hb_model_weight_bytes(model: *const hb_model, out: *mut u64) -> c_int;
        pub fn hb_model_set_softcap(model: *mut hb_model, softcap: f32) -> c_int;
        pub fn hb_model_set_precise_layers(model: *mut hb_model, n: c_int) -> c_int;
        pub fn hb_model_get_precise_layers(model: *const hb_model, out_n: *mut c_int) -> c_int;
        pub fn hb_model_upload_layer(
            model: *mut hb_model,
            layer: c_int,
            wq: *const f32,
            wk: *const f32,
            wv: *const f32,
            wo: *const f32,
            w1: *const f32,
            w3: *const f32,
            w2: *const f32,
            gamma1: *const f32,
            gamma2: *const f32,
        ) -> c_int;
        pub fn hb_model_upload_embed(model: *mut hb_model, embed: *const f32, gamma_final: *const f32) -> c_int;
        pub fn hb_model_init_synthetic(model: *mut hb_model, seed: u64, std: f32) -> c_int;

        // seeded synthetic inputs
        pub fn hb_synth_normal(seed: u64, tensor_id: u64, std: f32, n: u64, out: *mut f32) -> c_int;
        pub fn hb_synth_tokens(seed: u64, stream: u64, vocab: u32, n: u64, out: *mut u32) -> c_int;

        // forward (prefill)
        pub fn hb_forward(
            model: *mut hb_model,
            h_tokens: *const u32,
            h_targets: *const u32,
            b: c_int,
            s: c_int,
            h_per_pos_loss: *mut f32,
            h_logits: *mut f32,
            h_mean_loss: *mut f32,
        ) -> c_int;
        pub fn hb_forward_device(
            model: *mut hb_model,
            d_tokens: *const u32,
            d_targets: *const u32,
            b: c_int,
            s: c_int,
            d_per_pos_loss: *mut f32,
            d_logits: *mut f32,
            d_mean_loss: *mut f32,
        ) -> c_int;
        pub fn hb_model_reserve(model: *mut hb_model, b: c_int, s: c_int) -> c_int;
        pub fn hb_forward_timed(
            model: *mut hb_model,
            d_tokens: *const u32,
            d_targets: *const u32,
            b: c_int,
            s: c_int,
            d_per_pos_loss: *mut f32,
            d_mean_loss: *mut f32,
            out: *mut hb_forward_timings,
        ) -> c_int;

        // per-kernel entry points (device buffers)
        pub fn hb_op_rmsnorm(
            ctx: *mut hb_ctx,
            d_x: *const f32,
            d_gamma: *const f32,
            t: c_int,
            dim: c_int,
            eps: f32,
            d_out_f16: *mut c_void,
            d_rms_inv: *mut f32,
        ) -> c_int;
        pub fn hb_op_embedding(model: *mut hb_model, d_tokens: *const u32, t: c_int, d_x: *mut f32) -> c_int;
        pub fn hb_op_sdpa_fwd(
            model: *mut hb_model,
            layer: c_int,
            d_xnorm_f16: *const c_void,
            b: c_int,
            s: c_int,
            d_attn_f16: *mut c_void,
            d_qkv_tap: *mut f32,
        ) -> c_int;
        pub fn hb_op_wo_fwd(
            model: *mut hb_model,
            layer: c_int,
            d_attn_f16: *const c_void,
            d_x: *const f32,
            t: c_int,
            d_x2: *mut f32,
        ) -> c_int;
        pub fn hb_op_wo_fwd_noalloc(
            model: *mut hb_model,
            layer: c_int,
            d_attn_f16: *const c_void,
            d_x: *const f32,
            t: c_int,
            d_x2: *mut f32,
        ) -> c_int;
        pub fn hb_op_ffn_fused(
            model: *mut hb_model,
            layer: c_int,
            d_x2norm_f16: *const c_void,
            d_x2: *const f32,
            t: c_int,
            d_x_next: *mut f32,
            d_h13_tap: *mut f32,
            d_gate_f16: *mut c_void,
        ) -> c_int;
        pub fn hb_op_ffn_up(
            model: *mut hb_model,
            layer: c_int,
            d_x2norm_f16: *const c_void,
            t: c_int,
            d_gate_f16: *mut c_void,
            d_h13_tap: *mut f32,
        ) -> c_int;
        pub fn hb_op_logits_ce(
            model: *mut hb_model,
            d_xf_f16: *const c_void,
            d_targets: *const u32,
            t: c_int,
            d_logits: *mut f32,
            d_losses: *mut f32,
        ) -> c_int;
        pub fn hb_op_gemm_nt(
            ctx: *mut hb_ctx,
            d_a_f16: *const c_void,
            d_b_f16: *const c_void,
            d_c: *mut f32,
            m: c_int,
            n: c_int,
            k: c_int,
        ) -> c_int;

        // single-token decode
        pub fn hb_kv_create(model: *mut hb_model, batch: c_int, ctx_max: c_int, out: *mut *mut hb_kv) -> c_int;
        pub fn hb_kv_destroy(kv: *mut hb_kv) -> c_int;
        pub fn hb_kv_reset(kv: *mut hb_kv) -> c_int;
        pub fn hb_kv_length(kv: *mut hb_kv, out_len: *mut c_int) -> c_int;
        pub fn hb_kv_bytes(kv: *mut hb_kv, out: *mut u64) -> c_int;
        pub fn hb_prefill(
            model: *mut hb_model,
            kv: *mut hb_kv,
            h_tokens: *const u32,
            s: c_int,
            h_logits: *mut f32,
            h_next: *mut u32,
        ) -> c_int;
        pub fn hb_decode_step(
            model: *mut hb_model,
            kv: *mut hb_kv,
            h_tokens: *const u32,
            h_logits: *mut f32,
            h_next: *mut u32,
        ) -> c_int;
        pub fn hb_decode_greedy(
            model: *mut hb_model,
            kv: *mut hb_kv,
            h_first: *const u32,
            nsteps: c_int,
            h_out: *mut u32,
        ) -> c_int;

        // optimizer
        pub fn hb_learning_rate(tc: *const hb_train_config, step: u32, out_lr: *mut f32) -> c_int;
        pub fn hb_opt_create(model: *mut hb_model, tc: *const hb_train_config, out: *mut *mut hb_opt) -> c_int;
        pub fn hb_opt_destroy(opt: *mut hb_opt) -> c_int;
        pub fn hb_opt_upload_layer(
            opt: *mut hb_opt,
            layer: c_int,
            wq: *const f32,
            wk: *const f32,
            wv: *const f32,
            wo: *const f32,
            w1: *const f32,
            w3: *const f32,
            w2: *const f32,
            gamma1: *const f32,
            gamma2: *const f32,
        ) -> c_int;
        pub fn hb_opt_upload_embed(opt: *mut hb_opt, embed: *const f32, gamma_final: *const f32) -> c_int;
        pub fn hb_opt_init_synthetic(opt: *mut hb_opt, seed: u64, std: f32) -> c_int;
        pub fn hb_opt_upload_grads_layer(
            opt: *mut hb_opt,
            layer: c_int,
            dwq: *const f32,
            dwk: *const f32,
            dwv: *const f32,
            dwo: *const f32,
            dw1: *const f32,
            dw3: *const f32,
            dw2: *const f32,
            dgamma1: *const f32,
            dgamma2: *const f32,
        ) -> c_int;
        pub fn hb_opt_upload_grads_embed(opt: *mut hb_opt, dembed: *const f32, dgamma_final: *const f32) -> c_int;
        pub fn hb_opt_zero_grads(opt: *mut hb_opt) -> c_int;
        pub fn hb_opt_grad_arena(opt: *mut hb_opt, d_grads: *mut *mut f32, n_floats: *mut u64) -> c_int;
        pub fn hb_opt_grad_norm(opt: *mut hb_opt, out_norm: *mut f32) -> c_int;
        pub fn hb_opt_clip_grads(opt: *mut hb_opt, max_norm: f32, out_norm: *mut f32) -> c_int;
        pub fn hb_opt_update_weights(opt: *mut hb_opt, t: u32, lr: f32, grad_scale: f32) -> c_int;
        pub fn hb_opt_step(opt: *mut hb_opt, step: u32, out_norm: *mut f32) -> c_int;
        pub fn hb_opt_download_layer(
            opt: *mut hb_opt,
            layer: c_int,
            which: c_int,
            wq: *mut f32,
            wk: *mut f32,
            wv: *mut f32,
            wo: *mut f32,
            w1: *mut f32,
            w3: *mut f32,
            w2: *mut f32,
            gamma1: *mut f32,
            gamma2: *mut f32,
        ) -> c_int;
        pub fn hb_opt_download_embed(opt: *mut hb_opt, which: c_int, embed: *mut f32, gamma_final: *mut f32) -> c_int;

        // training forward + backward
        pub fn hb_forward_backward(
            m: *mut hb_model,
            opt: *mut hb_opt,
            tokens: *const u32,
            targets: *const u32,
            b: c_int,
            s: c_int,
            loss_scale: f32,
            per_pos_loss: *mut f32,
            mean_loss: *mut f32,
        ) -> c_int;
        pub fn hb_forward_backward_device(
            m: *mut hb_model,
            opt: *mut hb_opt,
            d_tokens: *const u32,
            d_targets: *const u32,
            b: c_int,
            s: c_int,
            loss_scale: f32,
            d_loss: *mut f32,
            d_mean: *mut f32,
        ) -> c_int;
        pub fn hb_train_forward(
            m: *mut hb_model,
            h_tokens: *const u32,
            h_targets: *const u32,
            b: c_int,
            s: c_int,
            h_per_pos_loss: *mut f32,
            h_mean_loss: *mut f32,
            out: *const hb_forward_result,
        ) -> c_int;
        pub fn hb_train_backward(m: *mut hb_model, opt: *mut hb_opt, loss_scale: f32) -> c_int;

        // RSTK checkpoints
        pub fn hb_rstk_read_header(path: *const c_char, out: *mut hb_rstk_header) -> c_int;
        pub fn hb_model_load_rstk(model: *mut hb_model, opt: *mut hb_opt, path: *const c_char, out_step: *mut u32) -> c_int;
        pub fn hb_model_save_rstk(model: *mut hb_model, opt: *mut hb_opt, step: u32, path: *const c_char) -> c_int;

        // data path and validation
        pub fn hb_tokens_create(ctx: *mut hb_ctx, h_tokens: *const u16, n: u64, out: *mut *mut hb_tokens) -> c_int;
        pub fn hb_tokens_open(ctx: *mut hb_ctx, path: *const c_char, out: *mut *mut hb_tokens) -> c_int;
        pub fn hb_tokens_destroy(t: *mut hb_tokens) -> c_int;
        pub fn hb_tokens_length(t: *const hb_tokens, out_n: *mut u64) -> c_int;
        pub fn hb_validate(
            model: *mut hb_model,
            val: *const hb_tokens,
            token_bytes: *const i32,
            tb_len: c_int,
            steps: c_int,
            batch: c_int,
            out_avg_loss: *mut f32,
            out_bpb: *mut f32,
            out_nats: *mut f64,
            out_bytes: *mut u64,
        ) -> c_int;

        // failure injection
        pub fn hb_debug_inject_error(code: c_int) -> c_int;
    }
}

// ---------------------------------------------------------------------------
// safe layer
// ---------------------------------------------------------------------------

/// A failed call: the HB_E_* code and the library's message for it.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct HbError {
    pub code: i32,
    pub message: String,
}

impl std::fmt::Display for HbError {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "hip-bridge error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for HbError {}

pub type Result<T> = std::result::Result<T, HbError>;

fn check(code: c_int) -> Result<()> {
    if code == sys::HB_OK {
        return Ok(());
    }
    // SAFETY: hb_last_error returns a valid, NUL-terminated thread-local string.
    let message = unsafe { CStr::from_ptr(sys::hb_last_error()) }.to_string_lossy().into_owned();
    Err(HbError { code, message })
}

fn invalid(message: String) -> HbError {
    HbError { code: sys::HB_E_INVALID, message }
}

fn need_len(what: &str, got: usize, want: usize) -> Result<()> {
    if got == want {
        Ok(())
    } else {
        Err(invalid(format!("{what}: {got} elements, expected {want}")))
    }
}

fn c_path(p: &Path) -> Result<CString> {
    CString::new(p.to_string_lossy().as_bytes()).map_err(|_| invalid("path contains a NUL byte".into()))
}

fn ptr_or_null<T>(s: Option<&mut [T]>) -> *mut T {
    s.map_or(ptr::null_mut(), |s| s.as_mut_ptr())
}

/// "hip-gfx950".
pub fn backend_name() -> &'static str {
    // SAFETY: a static NUL-terminated string owned by the library.
    unsafe { CStr::from_ptr(sys::hb_backend_name()) }.to_str().unwrap_or("")
}

pub fn device_count() -> Result<i32> {
    let mut n: c_int = 0;
    check(unsafe { sys::hb_device_count(&mut n) })?;
    Ok(n)
}

/// Model shape in the field names of the engine's ModelConfig (model.rs:5-17).
#[derive(Debug, Clone, Copy, PartialEq)]
pub struct ModelShape {
    pub dim: usize,
    pub hidden: usize,
    pub heads: usize,
    pub kv_heads: usize,
    pub hd: usize,
    pub seq: usize,
    pub nlayers: usize,
    pub vocab: usize,
    pub q_dim: usize,
    pub kv_dim: usize,
    pub gqa_ratio: usize,
    /// full_model.rs:234-239 (0 = off); the reference passes it per call.
    pub softcap: f32,
}

impl ModelShape {
    fn raw(&self) -> sys::hb_model_config {
        sys::hb_model_config {
            dim: self.dim as i32,
            hidden: self.hidden as i32,
            heads: self.heads as i32,
            kv_heads: self.kv_heads as i32,
            hd: self.hd as i32,
            seq: self.seq as i32,
            nlayers: self.nlayers as i32,
            vocab: self.vocab as i32,
            q_dim: self.q_dim as i32,
            kv_dim: self.kv_dim as i32,
            gqa_ratio: self.gqa_ratio as i32,
            rope_theta: 0.0,
            norm_eps: 0.0,
            residual_alpha: 0.0,
            softcap: self.softcap,
        }
    }

    /// hb_config_validate: the library's shape rules, no device needed.
    pub fn validate(&self) -> Result<()> {
        let mut c = self.raw();
        check(unsafe { sys::hb_config_validate(&mut c) })
    }
}

/// One device, one HIP stream (hb_ctx).
pub struct Context {
    raw: *mut sys::hb_ctx,
}

unsafe impl Send for Context {}

impl Context {
    pub fn new(device: i32) -> Result<Self> {
        let mut raw = ptr::null_mut();
        check(unsafe { sys::hb_ctx_create(device, &mut raw) })?;
        Ok(Context { raw })
    }

    pub fn synchronize(&self) -> Result<()> {
        check(unsafe { sys::hb_ctx_synchronize(self.raw) })
    }

    pub fn as_raw(&self) -> *mut sys::hb_ctx {
        self.raw
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        unsafe {
            sys::hb_ctx_destroy(self.raw);
        }
    }
}

/// One layer's fp32 weights in the reference layouts (LayerWeights, layer.rs:16-26).
pub struct LayerWeightsRef<'a> {
    pub wq: &'a [f32],
    pub wk: &'a [f32],
    pub wv: &'a [f32],
    pub wo: &'a [f32],
    pub w1: &'a [f32],
    pub w3: &'a [f32],
    pub w2: &'a [f32],
    pub gamma1: &'a [f32],
    pub gamma2: &'a [f32],
}

/// Per-position losses and optional logits of one forward.
pub struct ForwardOut {
    pub mean_loss: f32,
    pub losses: Vec<f32>,
    pub logits: Option<Vec<f32>>,
}

/// ForwardResult's host views (full_model.rs:73-81); the caches stay on the device.
#[derive(Debug, Default)]
pub struct ForwardViews {
    pub loss: f32,
    pub losses: Vec<f32>,
    pub dlogits: Vec<f32>,
    pub x_final: Vec<f32>,
    pub x_prenorm: Vec<f32>,
    pub rms_inv_final: Vec<f32>,
    pub logits_capped: Vec<f32>,
}

/// Device weights of one model (hb_model): what CompiledKernels::compile and
/// ModelWeights become on the GPU.
pub struct Model<'c> {
    raw: *mut sys::hb_model,
    cfg: sys::hb_model_config,
    _ctx: PhantomData<&'c Context>,
}

unsafe impl Send for Model<'_> {}

impl<'c> Model<'c> {
    pub fn new(ctx: &'c Context, shape: &ModelShape) -> Result<Self> {
        let c = shape.raw();
        let mut raw = ptr::null_mut();
        check(unsafe { sys::hb_model_create(ctx.raw, &c, sys::HB_DTYPE_F16, &mut raw) })?;
        let mut cfg = sys::hb_model_config::default();
        let r = check(unsafe { sys::hb_model_get_config(raw, &mut cfg) });
        let model = Model { raw, cfg, _ctx: PhantomData };
        r.map(|_| model)
    }

    pub fn config(&self) -> sys::hb_model_config {
        self.cfg
    }

    pub fn as_raw(&self) -> *mut sys::hb_model {
        self.raw
    }

    pub fn set_softcap(&mut self, softcap: f32) -> Result<()> {
        check(unsafe { sys::hb_model_set_softcap(self.raw, softcap) })?;
        self.cfg.softcap = softcap;
        Ok(())
    }

    /// hb_model_set_precise_layers: the first n layers of later forwards run
    /// on two-term fp16 operands (~22-bit inputs to their products).
    pub fn set_precise_layers(&mut self, n: usize) -> Result<()> {
        check(unsafe { sys::hb_model_set_precise_layers(self.raw, n as c_int) })
    }

    pub fn upload_layer(&mut self, layer: usize, w: &LayerWeightsRef<'_>) -> Result<()> {
        let c = &self.cfg;
        let (d, q, kv, h) = (c.dim as usize, c.q_dim as usize, c.kv_dim as usize, c.hidden as usize);
        need_len("wq", w.wq.len(), d * q)?;
        need_len("wk", w.wk.len(), d * kv)?;
        need_len("wv", w.wv.len(), d * kv)?;
        need_len("wo", w.wo.len(), q * d)?;
        need_len("w1", w.w1.len(), d * h)?;
        need_len("w3", w.w3.len(), d * h)?;
        need_len("w2", w.w2.len(), d * h)?;
        need_len("gamma1", w.gamma1.len(), d)?;
        need_len("gamma2", w.gamma2.len(), d)?;
        check(unsafe {
            sys::hb_model_upload_layer(
                self.raw,
                layer as c_int,
                w.wq.as_ptr(),
                w.wk.as_ptr(),
                w.wv.as_ptr(),
                w.wo.as_ptr(),
                w.w1.as_ptr(),
                w.w3.as_ptr(),
                w.w2.as_ptr(),
                w.gamma1.as_ptr(),
                w.gamma2.as_ptr(),
            )
        })
    }

    pub fn upload_embed(&mut self, embed: &[f32], gamma_final: &[f32]) -> Result<()> {
        let (v, d) = (self.cfg.vocab as usize, self.cfg.dim as usize);
        need_len("embed", embed.len(), v * d)?;
        need_len("gamma_final", gamma_final.len(), d)?;
        check(unsafe { sys::hb_model_upload_embed(self.raw, embed.as_ptr(), gamma_final.as_ptr()) })
    }

    pub fn init_synthetic(&mut self, seed: u64, std: f32) -> Result<()> {
        check(unsafe { sys::hb_model_init_synthetic(self.raw, seed, std) })
    }

    /// forward_ws / forward_losses (full_model.rs:187-247, 717-767) for
    /// `batch` sequences laid one after another in `tokens`.
    pub fn forward(&mut self, tokens: &[u32], targets: Option<&[u32]>, batch: usize, want_logits: bool) -> Result<ForwardOut> {
        if batch == 0 || tokens.len() % batch != 0 {
            return Err(invalid(format!("{} tokens do not split into {batch} sequences", tokens.len())));
        }
        let s = tokens.len() / batch;
        if let Some(t) = targets {
            need_len("targets", t.len(), tokens.len())?;
        }
        let mut losses = vec![0.0f32; if targets.is_some() { tokens.len() } else { 0 }];
        let mut logits = if want_logits { Some(vec![0.0f32; tokens.len() * self.cfg.vocab as usize]) } else { None };
        let mut mean = 0.0f32;
        check(unsafe {
            sys::hb_forward(
                self.raw,
                tokens.as_ptr(),
                targets.map_or(ptr::null(), |t| t.as_ptr()),
                batch as c_int,
                s as c_int,
                if targets.is_some() { losses.as_mut_ptr() } else { ptr::null_mut() },
                logits.as_mut().map_or(ptr::null_mut(), |l| l.as_mut_ptr()),
                if targets.is_some() { &mut mean as *mut f32 } else { ptr::null_mut() },
            )
        })?;
        Ok(ForwardOut { mean_loss: mean, losses, logits })
    }

    /// forward (full_model.rs:345-410) for training: the activations stay on
    /// the device for [`Optimizer::backward`]; the ForwardResult views come back.
    pub fn train_forward(&mut self, tokens: &[u32], targets: &[u32], batch: usize) -> Result<ForwardViews> {
        if batch == 0 || tokens.len() % batch != 0 {
            return Err(invalid(format!("{} tokens do not split into {batch} sequences", tokens.len())));
        }
        need_len("targets", targets.len(), tokens.len())?;
        let n = tokens.len();
        let (v, d) = (self.cfg.vocab as usize, self.cfg.dim as usize);
        let mut out = ForwardViews {
            loss: 0.0,
            losses: vec![0.0; n],
            dlogits: vec![0.0; n * v],
            x_final: vec![0.0; n * d],
            x_prenorm: vec![0.0; n * d],
            rms_inv_final: vec![0.0; n],
            logits_capped: if self.cfg.softcap > 0.0 { vec![0.0; n * v] } else { Vec::new() },
        };
        let views = sys::hb_forward_result {
            dlogits: out.dlogits.as_mut_ptr(),
            x_final: out.x_final.as_mut_ptr(),
            x_prenorm: out.x_prenorm.as_mut_ptr(),
            rms_inv_final: out.rms_inv_final.as_mut_ptr(),
            logits_capped: if out.logits_capped.is_empty() { ptr::null_mut() } else { out.logits_capped.as_mut_ptr() },
        };
        check(unsafe {
            sys::hb_train_forward(
                self.raw,
                tokens.as_ptr(),
                targets.as_ptr(),
                batch as c_int,
                (n / batch) as c_int,
                out.losses.as_mut_ptr(),
                &mut out.loss,
                &views,
            )
        })?;
        Ok(out)
    }

    pub fn load_rstk(&mut self, opt: Option<&mut Optimizer<'_, '_>>, path: &Path) -> Result<u32> {
        let p = c_path(path)?;
        let mut step = 0u32;
        let o = opt.map_or(ptr::null_mut(), |o| o.raw);
        check(unsafe { sys::hb_model_load_rstk(self.raw, o, p.as_ptr(), &mut step) })?;
        Ok(step)
    }

    pub fn save_rstk(&mut self, opt: Option<&mut Optimizer<'_, '_>>, step: u32, path: &Path) -> Result<()> {
        let p = c_path(path)?;
        let o = opt.map_or(ptr::null_mut(), |o| o.raw);
        check(unsafe { sys::hb_model_save_rstk(self.raw, o, step, p.as_ptr()) })
    }
}

impl Drop for Model<'_> {
    fn drop(&mut self) {
        unsafe {
            sys::hb_model_destroy(self.raw);
        }
    }
}

/// Preallocated fp16 KV cache and decode state for `batch` sequences (hb_kv).
pub struct KvCache<'m, 'c> {
    raw: *mut sys::hb_kv,
    batch: usize,
    vocab: usize,
    _model: PhantomData<&'m Model<'c>>,
}

unsafe impl Send for KvCache<'_, '_> {}

impl<'m, 'c> KvCache<'m, 'c> {
    pub fn new(model: &'m Model<'c>, batch: usize, ctx_max: usize) -> Result<Self> {
        let mut raw = ptr::null_mut();
        check(unsafe { sys::hb_kv_create(model.raw, batch as c_int, ctx_max as c_int, &mut raw) })?;
        Ok(KvCache { raw, batch, vocab: model.cfg.vocab as usize, _model: PhantomData })
    }

    pub fn len(&self) -> Result<usize> {
        let mut n: c_int = 0;
        check(unsafe { sys::hb_kv_length(self.raw, &mut n) })?;
        Ok(n as usize)
    }

    pub fn is_empty(&self) -> Result<bool> {
        Ok(self.len()? == 0)
    }

    pub fn reset(&mut self) -> Result<()> {
        check(unsafe { sys::hb_kv_reset(self.raw) })
    }

    /// Prompt of `batch` sequences of equal length; returns (last logits [batch*vocab], next tokens).
    pub fn prefill(&mut self, model: &mut Model<'c>, tokens: &[u32]) -> Result<(Vec<f32>, Vec<u32>)> {
        if tokens.is_empty() || tokens.len() % self.batch != 0 {
            return Err(invalid(format!("{} tokens do not split into {} sequences", tokens.len(), self.batch)));
        }
        let mut logits = vec![0.0f32; self.batch * self.vocab];
        let mut next = vec![0u32; self.batch];
        check(unsafe {
            sys::hb_prefill(
                model.raw,
                self.raw,
                tokens.as_ptr(),
                (tokens.len() / self.batch) as c_int,
                logits.as_mut_ptr(),
                next.as_mut_ptr(),
            )
        })?;
        Ok((logits, next))
    }

    /// One token per sequence at the current length.
    pub fn step(&mut self, model: &mut Model<'c>, tokens: &[u32], logits: Option<&mut [f32]>) -> Result<Vec<u32>> {
        need_len("tokens", tokens.len(), self.batch)?;
        if let Some(l) = &logits {
            need_len("logits", l.len(), self.batch * self.vocab)?;
        }
        let mut next = vec![0u32; self.batch];
        check(unsafe {
            sys::hb_decode_step(model.raw, self.raw, tokens.as_ptr(), ptr_or_null(logits), next.as_mut_ptr())
        })?;
        Ok(next)
    }

    /// `nsteps` greedy steps on the device; returns the generated tokens [nsteps*batch].
    pub fn greedy(&mut self, model: &mut Model<'c>, first: &[u32], nsteps: usize) -> Result<Vec<u32>> {
        need_len("first", first.len(), self.batch)?;
        let mut out = vec![0u32; nsteps * self.batch];
        check(unsafe { sys::hb_decode_greedy(model.raw, self.raw, first.as_ptr(), nsteps as c_int, out.as_mut_ptr()) })?;
        Ok(out)
    }
}

impl Drop for KvCache<'_, '_> {
    fn drop(&mut self) {
        unsafe {
            sys::hb_kv_destroy(self.raw);
        }
    }
}

/// ModelOptState + ModelGrads on the device (hb_opt).
pub struct Optimizer<'m, 'c> {
    raw: *mut sys::hb_opt,
    model: *mut sys::hb_model,
    _model: PhantomData<&'m Model<'c>>,
}

unsafe impl Send for Optimizer<'_, '_> {}

impl<'m, 'c> Optimizer<'m, 'c> {
    pub fn new(model: &'m Model<'c>, tc: &sys::hb_train_config) -> Result<Self> {
        let mut raw = ptr::null_mut();
        check(unsafe { sys::hb_opt_create(model.raw, tc, &mut raw) })?;
        Ok(Optimizer { raw, model: model.raw, _model: PhantomData })
    }

    pub fn zero_grads(&mut self) -> Result<()> {
        check(unsafe { sys::hb_opt_zero_grads(self.raw) })
    }

    /// forward_ws + backward_ws (full_model.rs:187-331): gradients of
    /// loss_scale * mean CE added to the arena; returns the mean loss.
    pub fn forward_backward(&mut self, tokens: &[u32], targets: &[u32], batch: usize, loss_scale: f32) -> Result<f32> {
        if batch == 0 || tokens.len() % batch != 0 {
            return Err(invalid(format!("{} tokens do not split into {batch} sequences", tokens.len())));
        }
        need_len("targets", targets.len(), tokens.len())?;
        let mut mean = 0.0f32;
        check(unsafe {
            sys::hb_forward_backward(
                self.model,
                self.raw,
                tokens.as_ptr(),
                targets.as_ptr(),
                batch as c_int,
                (tokens.len() / batch) as c_int,
                loss_scale,
                ptr::null_mut(),
                &mut mean,
            )
        })?;
        Ok(mean)
    }

    /// backward (full_model.rs:414-483) from the model's last Model::train_forward.
    pub fn backward(&mut self, loss_scale: f32) -> Result<()> {
        check(unsafe { sys::hb_train_backward(self.model, self.raw, loss_scale) })
    }

    pub fn grad_norm(&mut self) -> Result<f32> {
        let mut n = 0.0f32;
        check(unsafe { sys::hb_opt_grad_norm(self.raw, &mut n) })?;
        Ok(n)
    }

    /// The optimizer half of train_step (full_model.rs:697-711); returns the raw norm.
    pub fn step(&mut self, step: u32) -> Result<f32> {
        let mut n = 0.0f32;
        check(unsafe { sys::hb_opt_step(self.raw, step, &mut n) })?;
        Ok(n)
    }
}

impl Drop for Optimizer<'_, '_> {
    fn drop(&mut self) {
        unsafe {
            sys::hb_opt_destroy(self.raw);
        }
    }
}

/// TokenData (data.rs:11-40) resident on the device (hb_tokens).
pub struct TokenStream<'c> {
    raw: *mut sys::hb_tokens,
    _ctx: PhantomData<&'c Context>,
}

impl<'c> TokenStream<'c> {
    pub fn open(ctx: &'c Context, path: &Path) -> Result<Self> {
        let p = c_path(path)?;
        let mut raw = ptr::null_mut();
        check(unsafe { sys::hb_tokens_open(ctx.raw, p.as_ptr(), &mut raw) })?;
        Ok(TokenStream { raw, _ctx: PhantomData })
    }

    pub fn from_slice(ctx: &'c Context, tokens: &[u16]) -> Result<Self> {
        let mut raw = ptr::null_mut();
        check(unsafe { sys::hb_tokens_create(ctx.raw, tokens.as_ptr(), tokens.len() as u64, &mut raw) })?;
        Ok(TokenStream { raw, _ctx: PhantomData })
    }

    /// validate (bin/train.rs:123-163): (mean loss, val_bpb).
    pub fn validate(&self, model: &mut Model<'c>, token_bytes: Option<&[i32]>, steps: usize, batch: usize) -> Result<(f32, f32)> {
        let (mut avg, mut bpb) = (0.0f32, 0.0f32);
        let (tb, tb_len) = token_bytes.map_or((ptr::null(), 0), |t| (t.as_ptr(), t.len() as c_int));
        check(unsafe {
            sys::hb_validate(
                model.raw,
                self.raw,
                tb,
                tb_len,
                steps as c_int,
                batch as c_int,
                &mut avg,
                &mut bpb,
                ptr::null_mut(),
                ptr::null_mut(),
            )
        })?;
        Ok((avg, bpb))
    }
}

impl Drop for TokenStream<'_> {
    fn drop(&mut self) {
        unsafe {
            sys::hb_tokens_destroy(self.raw);
        }
    }
}

/// Seeded N(0, std^2) values (host, deterministic), as hb_model_init_synthetic fills them.
pub fn synth_normal(seed: u64, tensor_id: u64, std: f32, n: usize) -> Result<Vec<f32>> {
    let mut out = vec![0.0f32; n];
    check(unsafe { sys::hb_synth_normal(seed, tensor_id, std, n as u64, out.as_mut_ptr()) })?;
    Ok(out)
}

/// Last error message on this thread ("" if none).
pub fn last_error() -> String {
    unsafe { CStr::from_ptr(sys::hb_last_error()) }.to_string_lossy().into_owned()
}
