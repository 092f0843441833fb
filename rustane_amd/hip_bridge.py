"""ctypes binding of libhip_bridge.so (include/hip_bridge.h).

This is the Python counterpart of the `hip-bridge` crate that replaces rustane's
`ane-bridge` (crates/ane-bridge/src/lib.rs:8-9): a thin, typed wrapper over the
C ABI. Errors come back as :class:`HipBridgeError` carrying the library's code
and message, where the reference panicked with ``.expect("ANE eval failed")``
(crates/engine/src/layer.rs:727).

The library is loaded from the package directory only; there is no fallback
implementation. If ``libhip_bridge.so`` is missing, :func:`lib` raises.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import threading
from dataclasses import dataclass, fields

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhip_bridge.so")

HB_OK = 0
HB_E_INVALID = -1
HB_E_CONFIG = -2
HB_E_DEVICE = -3
HB_E_OOM = -4
HB_E_STATE = -5
HB_E_INJECTED = -6
HB_DTYPE_F16 = 1
HB_SYNTH_EMBED_ID = 0xFFFF

_CODE_NAMES = {
    HB_E_INVALID: "HB_E_INVALID",
    HB_E_CONFIG: "HB_E_CONFIG",
    HB_E_DEVICE: "HB_E_DEVICE",
    HB_E_OOM: "HB_E_OOM",
    HB_E_STATE: "HB_E_STATE",
    HB_E_INJECTED: "HB_E_INJECTED",
}


class HipBridgeError(RuntimeError):
    def __init__(self, code: int, msg: str, func: str):
        self.code = code
        super().__init__(f"{func}: {_CODE_NAMES.get(code, code)}: {msg}")


class hb_model_config(C.Structure):
    _fields_ = [
        ("dim", C.c_int32),
        ("hidden", C.c_int32),
        ("heads", C.c_int32),
        ("kv_heads", C.c_int32),
        ("hd", C.c_int32),
        ("seq", C.c_int32),
        ("nlayers", C.c_int32),
        ("vocab", C.c_int32),
        ("q_dim", C.c_int32),
        ("kv_dim", C.c_int32),
        ("gqa_ratio", C.c_int32),
        ("rope_theta", C.c_float),
        ("norm_eps", C.c_float),
        ("residual_alpha", C.c_float),
        ("softcap", C.c_float),
    ]


class hb_train_config(C.Structure):
    """TrainConfig (full_model.rs:33-70), the optimizer's fields."""
    _fields_ = [
        ("max_lr", C.c_float),
        ("min_lr_frac", C.c_float),
        ("warmup_steps", C.c_uint32),
        ("total_steps", C.c_uint32),
        ("beta1", C.c_float),
        ("beta2", C.c_float),
        ("eps", C.c_float),
        ("weight_decay", C.c_float),
        ("matrix_lr_scale", C.c_float),
        ("embed_lr_scale", C.c_float),
        ("loss_scale", C.c_float),
        ("accum_steps", C.c_uint32),
        ("grad_clip", C.c_float),
    ]


class hb_forward_result(C.Structure):
    """ForwardResult's host views (full_model.rs:73-81); each pointer nullable."""
    _fields_ = [(n, C.c_void_p) for n in ("dlogits", "x_final", "x_prenorm", "rms_inv_final",
                                          "logits_capped")]


class hb_forward_timings(C.Structure):
    """Per-stage device time of one forward (ForwardTimings, layer.rs:821-1015):
    stage sums over layers 1..nlayers-1, the first layer in layer0_ms."""
    _fields_ = [(n, C.c_float) for n in (
        "embedding_ms", "rmsnorm1_ms", "sdpa_qkv_ms", "sdpa_attention_ms", "wo_ms", "residual_rmsnorm2_ms",
        "ffn_up_ms", "ffn_down_ms", "ffn_residual_norm_ms", "logits_ms", "cross_entropy_ms", "layer0_ms",
        "total_ms")] + [("layers_summed", C.c_int32)]

    def as_dict(self) -> dict:
        return {n: getattr(self, n) for n, _ in self._fields_}


class hb_rstk_header(C.Structure):
    """RSTK checkpoint header (bin/train.rs:175-183) after the magic."""
    _fields_ = [(n, C.c_uint32) for n in ("version", "step", "dim", "nlayers", "vocab", "seq")]


_P = C.c_void_p
_I = C.c_int
_F = C.c_float
_U64 = C.c_uint64
_U32 = C.c_uint32
_FP = C.POINTER(C.c_float)
_UP = C.POINTER(C.c_uint32)

# name -> argtypes; every function returns int status unless listed in _RESTYPE.
SIGNATURES = {
    "hb_backend_name": [],
    "hb_last_error": [],
    "hb_device_count": [C.POINTER(C.c_int)],
    "hb_ctx_create": [_I, C.POINTER(_P)],
    "hb_ctx_destroy": [_P],
    "hb_ctx_set_stream": [_P, _P],
    "hb_ctx_get_stream": [_P, C.POINTER(_P)],
    "hb_ctx_synchronize": [_P],
    "hb_model_create": [_P, C.POINTER(hb_model_config), _I, C.POINTER(_P)],
    "hb_model_destroy": [_P],
    "hb_config_validate": [C.POINTER(hb_model_config)],
    "hb_model_get_config": [_P, C.POINTER(hb_model_config)],
    "hb_model_weight_bytes": [_P, C.POINTER(C.c_uint64)],
    "hb_model_set_softcap": [_P, _F],
    "hb_model_set_precise_layers": [_P, _I],
    "hb_model_get_precise_layers": [_P, C.POINTER(C.c_int)],
    "hb_model_upload_layer": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "hb_model_upload_embed": [_P, _P, _P],
    "hb_model_init_synthetic": [_P, _U64, _F],
    "hb_synth_normal": [_U64, _U64, _F, _U64, _P],
    "hb_synth_tokens": [_U64, _U64, _U32, _U64, _P],
    "hb_forward": [_P, _P, _P, _I, _I, _P, _P, _P],
    "hb_forward_device": [_P, _P, _P, _I, _I, _P, _P, _P],
    "hb_model_reserve": [_P, _I, _I],
    "hb_forward_timed": [_P, _P, _P, _I, _I, _P, _P, _P],
    "hb_op_rmsnorm": [_P, _P, _P, _I, _I, _F, _P, _P],
    "hb_op_embedding": [_P, _P, _I, _P],
    "hb_op_sdpa_fwd": [_P, _I, _P, _I, _I, _P, _P],
    "hb_op_wo_fwd": [_P, _I, _P, _P, _I, _P],
    "hb_op_wo_fwd_noalloc": [_P, _I, _P, _P, _I, _P],
    "hb_op_ffn_fused": [_P, _I, _P, _P, _I, _P, _P, _P],
    "hb_op_ffn_up": [_P, _I, _P, _I, _P, _P],
    "hb_op_logits_ce": [_P, _P, _P, _I, _P, _P],
    "hb_op_gemm_nt": [_P, _P, _P, _P, _I, _I, _I],
    "hb_kv_create": [_P, _I, _I, C.POINTER(_P)],
    "hb_kv_destroy": [_P],
    "hb_kv_reset": [_P],
    "hb_kv_length": [_P, C.POINTER(C.c_int)],
    "hb_kv_bytes": [_P, C.POINTER(C.c_uint64)],
    "hb_prefill": [_P, _P, _P, _I, _P, _P],
    "hb_decode_step": [_P, _P, _P, _P, _P],
    "hb_decode_greedy": [_P, _P, _P, _I, _P],
    "hb_learning_rate": [C.POINTER(hb_train_config), _U32, C.POINTER(C.c_float)],
    "hb_opt_create": [_P, C.POINTER(hb_train_config), C.POINTER(_P)],
    "hb_opt_destroy": [_P],
    "hb_opt_upload_layer": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "hb_opt_upload_embed": [_P, _P, _P],
    "hb_opt_init_synthetic": [_P, _U64, _F],
    "hb_opt_upload_grads_layer": [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "hb_opt_upload_grads_embed": [_P, _P, _P],
    "hb_opt_zero_grads": [_P],
    "hb_opt_grad_arena": [_P, C.POINTER(_P), C.POINTER(C.c_uint64)],
    "hb_opt_grad_norm": [_P, C.POINTER(C.c_float)],
    "hb_opt_clip_grads": [_P, _F, C.POINTER(C.c_float)],
    "hb_opt_update_weights": [_P, _U32, _F, _F],
    "hb_opt_step": [_P, _U32, C.POINTER(C.c_float)],
    "hb_opt_download_layer": [_P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "hb_opt_download_embed": [_P, _I, _P, _P],
    "hb_forward_backward": [_P, _P, _P, _P, _I, _I, _F, _P, _P],
    "hb_forward_backward_device": [_P, _P, _P, _P, _I, _I, _F, _P, _P],
    "hb_train_forward": [_P, _P, _P, _I, _I, _P, _P, C.POINTER(hb_forward_result)],
    "hb_train_backward": [_P, _P, _F],
    "hb_rstk_read_header": [C.c_char_p, C.POINTER(hb_rstk_header)],
    "hb_model_load_rstk": [_P, _P, C.c_char_p, C.POINTER(C.c_uint32)],
    "hb_model_save_rstk": [_P, _P, _U32, C.c_char_p],
    "hb_tokens_create": [_P, _P, _U64, C.POINTER(_P)],
    "hb_tokens_open": [_P, C.c_char_p, C.POINTER(_P)],
    "hb_tokens_destroy": [_P],
    "hb_tokens_length": [_P, C.POINTER(C.c_uint64)],
    "hb_validate": [_P, _P, _P, _I, _I, _I, C.POINTER(C.c_float), C.POINTER(C.c_float),
                    C.POINTER(C.c_double), C.POINTER(C.c_uint64)],
    "hb_debug_inject_error": [_I],
}
_RESTYPE = {"hb_backend_name": C.c_char_p, "hb_last_error": C.c_char_p}

_lib = None
_lock = threading.Lock()
_exiting = False


def _mark_exiting():
    # After interpreter exit has begun, torch may already have released the
    # streams a context was bound to; the process is about to free all device
    # memory anyway, so finalizers stop calling into the library.
    global _exiting
    _exiting = True


atexit.register(_mark_exiting)


def lib() -> C.CDLL:
    """Load libhip_bridge.so (once). Raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise FileNotFoundError(
                    f"{LIB_PATH} not built: run `make -C rustane_amd/csrc` or "
                    "`python -c 'import __graft_entry__ as g; g.build()'`")
            L = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
            for name, argtypes in SIGNATURES.items():
                f = getattr(L, name)
                f.argtypes = argtypes
                f.restype = _RESTYPE.get(name, C.c_int)
            _lib = L
        return _lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != HB_OK:
        msg = lib().hb_last_error().decode(errors="replace")
        raise HipBridgeError(rc, msg, name)


def last_error() -> str:
    return lib().hb_last_error().decode(errors="replace")


def backend_name() -> str:
    return lib().hb_backend_name().decode()


def device_count() -> int:
    n = C.c_int(0)
    call("hb_device_count", C.byref(n))
    return n.value


def ptr(a) -> int | None:
    """Address of a numpy array or torch tensor (None passes through as NULL)."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data


def config_struct(cfg) -> hb_model_config:
    s = hb_model_config()
    for f in fields(hb_model_config_fields):
        setattr(s, f.name, getattr(cfg, f.name))
    return s


@dataclass
class hb_model_config_fields:
    dim: int
    hidden: int
    heads: int
    kv_heads: int
    hd: int
    seq: int
    nlayers: int
    vocab: int
    q_dim: int
    kv_dim: int
    gqa_ratio: int
    rope_theta: float
    norm_eps: float
    residual_alpha: float
    softcap: float


# ---- object wrappers ---------------------------------------------------------

class Context:
    """hb_ctx: one device + one HIP stream. Single owner, like CompiledKernels."""

    def __init__(self, device: int = 0):
        h = _P()
        call("hb_ctx_create", device, C.byref(h))
        self.handle = h
        self.device = device

    def set_stream(self, stream_ptr: int | None) -> None:
        call("hb_ctx_set_stream", self.handle, stream_ptr)

    def stream(self) -> int:
        s = _P()
        call("hb_ctx_get_stream", self.handle, C.byref(s))
        return s.value or 0

    def synchronize(self) -> None:
        call("hb_ctx_synchronize", self.handle)

    def close(self) -> None:
        if self.handle and not _exiting:
            lib().hb_ctx_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """hb_model: device weights for one ModelConfig."""

    def __init__(self, ctx: Context, cfg):
        h = _P()
        s = config_struct(cfg)
        call("hb_model_create", ctx.handle, C.byref(s), HB_DTYPE_F16, C.byref(h))
        self.handle = h
        self.ctx = ctx
        out = hb_model_config()
        call("hb_model_get_config", h, C.byref(out))
        self.config = out

    def upload_layer(self, layer: int, lw) -> None:
        import numpy as np
        arrs = [np.ascontiguousarray(getattr(lw, n), dtype=np.float32)
                for n in ("wq", "wk", "wv", "wo", "w1", "w3", "w2", "gamma1", "gamma2")]
        call("hb_model_upload_layer", self.handle, layer, *[a.ctypes.data for a in arrs])

    def upload_embed(self, embed, gamma_final) -> None:
        import numpy as np
        e = np.ascontiguousarray(embed, dtype=np.float32)
        g = np.ascontiguousarray(gamma_final, dtype=np.float32)
        call("hb_model_upload_embed", self.handle, e.ctypes.data, g.ctypes.data)

    def init_synthetic(self, seed: int, std: float = 0.02) -> None:
        call("hb_model_init_synthetic", self.handle, seed, std)

    def weight_bytes(self) -> int:
        n = C.c_uint64()
        call("hb_model_weight_bytes", self.handle, C.byref(n))
        return n.value

    def reserve(self, B: int, S: int) -> None:
        call("hb_model_reserve", self.handle, B, S)

    def forward_timed(self, d_tokens: int, d_targets, B: int, S: int, d_loss=None, d_mean=None) -> dict:
        """hb_forward_timed on device buffers (addresses): per-stage device times in ms."""
        t = hb_forward_timings()
        call("hb_forward_timed", self.handle, d_tokens, d_targets, B, S, d_loss, d_mean, C.byref(t))
        return t.as_dict()

    def set_precise_layers(self, n: int) -> None:
        """hb_model_set_precise_layers: the first n layers run on two-term fp16 operands."""
        call("hb_model_set_precise_layers", self.handle, n)

    def precise_layers(self) -> int:
        n = C.c_int()
        call("hb_model_get_precise_layers", self.handle, C.byref(n))
        return n.value

    def train_forward(self, tokens, targets, batch: int, seq: int, views=()):
        """hb_train_forward: the training forward of `batch` sequences of `seq`
        tokens, its activations kept on the device for the next backward.
        `views` names the ForwardResult fields to download (dlogits, x_final,
        x_prenorm, rms_inv_final, logits_capped). Returns (mean loss,
        per-position losses, {name: array})."""
        import numpy as np
        c = self.config
        tok = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        tgt = np.ascontiguousarray(targets, dtype=np.uint32).reshape(-1)
        n = batch * seq
        if tok.size != n or tgt.size != n:
            raise ValueError(f"expected {n} tokens and targets")
        shapes = {"dlogits": (n * c.vocab,), "logits_capped": (n * c.vocab,), "rms_inv_final": (n,),
                  "x_final": (batch, c.dim, seq), "x_prenorm": (batch, c.dim, seq)}
        out = {k: np.zeros(shapes[k], np.float32) for k in views}
        r = hb_forward_result(**{k: v.ctypes.data for k, v in out.items()})
        mean = C.c_float()
        losses = np.empty(n, np.float32)
        call("hb_train_forward", self.handle, tok.ctypes.data, tgt.ctypes.data, batch, seq,
             losses.ctypes.data, C.byref(mean), C.byref(r))
        return mean.value, losses, out

    def close(self) -> None:
        if self.handle and not _exiting:
            lib().hb_model_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class KVCache:
    """hb_kv: preallocated fp16 KV cache + decode state for `batch` sequences."""

    def __init__(self, model: Model, batch: int, ctx_max: int):
        h = _P()
        call("hb_kv_create", model.handle, batch, ctx_max, C.byref(h))
        self.handle = h
        self.model = model
        self.batch = batch
        self.ctx_max = ctx_max

    def length(self) -> int:
        n = C.c_int()
        call("hb_kv_length", self.handle, C.byref(n))
        return n.value

    def nbytes(self) -> int:
        n = C.c_uint64()
        call("hb_kv_bytes", self.handle, C.byref(n))
        return n.value

    def reset(self) -> None:
        call("hb_kv_reset", self.handle)

    def close(self) -> None:
        if self.handle and not _exiting:
            lib().hb_kv_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def synth_normal(seed: int, tensor_id: int, n: int, std: float = 0.02):
    import numpy as np
    out = np.empty(n, dtype=np.float32)
    call("hb_synth_normal", seed, tensor_id, std, n, out.ctypes.data)
    return out


def synth_tokens(seed: int, stream: int, vocab: int, n: int):
    import numpy as np
    out = np.empty(n, dtype=np.uint32)
    call("hb_synth_tokens", seed, stream, vocab, n, out.ctypes.data)
    return out


def train_config_struct(tc) -> hb_train_config:
    s = hb_train_config()
    for name, _ in hb_train_config._fields_:
        setattr(s, name, getattr(tc, name))
    return s


LAYER_TENSORS = ("wq", "wk", "wv", "wo", "w1", "w3", "w2", "gamma1", "gamma2")


class Optimizer:
    """hb_opt: fp32 master weights, gradients and AdamW moments of a Model on
    its device (ModelOptState + ModelGrads, full_model.rs:20-31)."""

    WEIGHTS, M, V, GRADS = 0, 1, 2, 3

    def __init__(self, model: Model, tc):
        self.model = model
        self.cfg = model.config
        self.tc = train_config_struct(tc)
        h = _P()
        call("hb_opt_create", model.handle, C.byref(self.tc), C.byref(h))
        self.handle = h

    def _layer_shapes(self):
        c = self.cfg
        d, q, kv, h = c.dim, c.q_dim, c.kv_dim, c.hidden
        return dict(wq=d * q, wk=d * kv, wv=d * kv, wo=q * d, w1=d * h, w3=d * h, w2=d * h,
                    gamma1=d, gamma2=d)

    @staticmethod
    def _arrays(obj, names):
        out = []
        for n in names:
            a = np.ascontiguousarray(getattr(obj, n), dtype=np.float32)
            out.append(a)
        return out

    def upload_layer(self, layer: int, lw) -> None:
        arrs = self._arrays(lw, LAYER_TENSORS)
        call("hb_opt_upload_layer", self.handle, layer, *[a.ctypes.data for a in arrs])

    def upload_embed(self, embed, gamma_final) -> None:
        e = np.ascontiguousarray(embed, dtype=np.float32)
        g = np.ascontiguousarray(gamma_final, dtype=np.float32)
        call("hb_opt_upload_embed", self.handle, e.ctypes.data, g.ctypes.data)

    def init_synthetic(self, seed: int, std: float = 0.02) -> None:
        call("hb_opt_init_synthetic", self.handle, seed, std)

    def upload_grads_layer(self, layer: int, grads: dict) -> None:
        arrs = [np.ascontiguousarray(grads[k], dtype=np.float32) for k in LAYER_TENSORS]
        call("hb_opt_upload_grads_layer", self.handle, layer, *[a.ctypes.data for a in arrs])

    def upload_grads_embed(self, dembed, dgamma_final) -> None:
        e = np.ascontiguousarray(dembed, dtype=np.float32)
        g = np.ascontiguousarray(dgamma_final, dtype=np.float32)
        call("hb_opt_upload_grads_embed", self.handle, e.ctypes.data, g.ctypes.data)

    def zero_grads(self) -> None:
        call("hb_opt_zero_grads", self.handle)

    def grad_arena(self):
        p, n = _P(), C.c_uint64()
        call("hb_opt_grad_arena", self.handle, C.byref(p), C.byref(n))
        return p.value, n.value

    def grad_norm(self) -> float:
        out = C.c_float()
        call("hb_opt_grad_norm", self.handle, C.byref(out))
        return out.value

    def clip_grads(self, max_norm: float) -> float:
        out = C.c_float()
        call("hb_opt_clip_grads", self.handle, max_norm, C.byref(out))
        return out.value

    def update_weights(self, t: int, lr: float, grad_scale: float) -> None:
        call("hb_opt_update_weights", self.handle, t, lr, grad_scale)

    def step(self, step: int, want_norm: bool = True):
        out = C.c_float()
        call("hb_opt_step", self.handle, step, C.byref(out) if want_norm else None)
        return out.value if want_norm else None

    def forward_backward(self, tokens, targets, batch: int, seq: int, loss_scale: float = 256.0,
                         want_losses: bool = False):
        """forward_ws + backward_ws (full_model.rs:187-331) of `batch`
        sequences of `seq` tokens: the gradients of loss_scale * mean CE of
        each sequence are ADDED to the gradient arena. Returns the mean loss
        over all positions (and the per-position losses)."""
        tok = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        tgt = np.ascontiguousarray(targets, dtype=np.uint32).reshape(-1)
        n = batch * seq
        if tok.size != n or tgt.size != n:
            raise ValueError(f"expected {n} tokens and targets")
        mean = C.c_float()
        losses = np.empty(n, np.float32) if want_losses else None
        call("hb_forward_backward", self.model.handle, self.handle, tok.ctypes.data, tgt.ctypes.data,
             batch, seq, loss_scale, losses.ctypes.data if want_losses else None, C.byref(mean))
        return (mean.value, losses) if want_losses else mean.value

    def backward(self, loss_scale: float = 256.0) -> None:
        """hb_train_backward: the backward of the model's last hb_train_forward,
        added to this optimizer's gradient arena."""
        call("hb_train_backward", self.model.handle, self.handle, loss_scale)

    def forward_backward_device(self, d_tokens: int, d_targets: int, batch: int, seq: int,
                                loss_scale: float = 256.0, d_loss: int = 0, d_mean: int = 0) -> None:
        """As forward_backward with the ids already in device memory (stream-ordered, no sync)."""
        call("hb_forward_backward_device", self.model.handle, self.handle, d_tokens, d_targets,
             batch, seq, loss_scale, d_loss or None, d_mean or None)

    def download_layer(self, layer: int, which: int = 0) -> dict:
        sh = self._layer_shapes()
        out = {k: np.empty(sh[k], np.float32) for k in LAYER_TENSORS}
        call("hb_opt_download_layer", self.handle, layer, which,
             *[out[k].ctypes.data for k in LAYER_TENSORS])
        return out

    def download_embed(self, which: int = 0):
        c = self.cfg
        e = np.empty(c.vocab * c.dim, np.float32)
        g = np.empty(c.dim, np.float32)
        call("hb_opt_download_embed", self.handle, which, e.ctypes.data, g.ctypes.data)
        return e, g

    def close(self) -> None:
        if self.handle and not _exiting:
            lib().hb_opt_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def learning_rate(tc, step: int) -> float:
    out = C.c_float()
    s = train_config_struct(tc)
    call("hb_learning_rate", C.byref(s), step, C.byref(out))
    return out.value


def rstk_read_header(path) -> dict:
    h = hb_rstk_header()
    call("hb_rstk_read_header", os.fsencode(path), C.byref(h))
    return {n: getattr(h, n) for n, _ in hb_rstk_header._fields_}


def rstk_load(model: Model, path, opt: "Optimizer | None" = None) -> int:
    step = C.c_uint32()
    call("hb_model_load_rstk", model.handle, opt.handle if opt else None, os.fsencode(path),
         C.byref(step))
    return step.value


def rstk_save(model: Model, path, step: int, opt: "Optimizer | None" = None) -> None:
    call("hb_model_save_rstk", model.handle, opt.handle if opt else None, step, os.fsencode(path))


class DeviceTokens:
    """hb_tokens: a uint16 token stream resident on the device."""

    def __init__(self, ctx: Context, tokens=None, path=None):
        h = _P()
        if path is not None:
            call("hb_tokens_open", ctx.handle, os.fsencode(path), C.byref(h))
        else:
            a = np.ascontiguousarray(tokens, dtype="<u2")
            call("hb_tokens_create", ctx.handle, a.ctypes.data if a.size else None, a.size, C.byref(h))
        self.handle = h

    def __len__(self) -> int:
        n = C.c_uint64()
        call("hb_tokens_length", self.handle, C.byref(n))
        return n.value

    def close(self) -> None:
        if self.handle and not _exiting:
            lib().hb_tokens_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def validate(model: Model, val: DeviceTokens, token_bytes, steps: int, batch: int = 1):
    """hb_validate -> (avg_loss, bpb, total_nats, total_bytes)."""
    tb = None if token_bytes is None else np.ascontiguousarray(token_bytes, dtype="<i4")
    avg, bpb, nats, nbytes = C.c_float(), C.c_float(), C.c_double(), C.c_uint64()
    call("hb_validate", model.handle, val.handle, tb.ctypes.data if tb is not None else None,
         tb.size if tb is not None else 0, steps, batch, C.byref(avg), C.byref(bpb), C.byref(nats),
         C.byref(nbytes))
    return avg.value, bpb.value, nats.value, nbytes.value
