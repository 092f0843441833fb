"""Model-level API of rustane's engine crate, served by libhip_bridge.

Mirrors the names and argument meaning of the reference so callers switch
without changes:

  ModelConfig        crates/engine/src/model.rs:5-152 (fields, presets, param_count)
  LayerWeights       crates/engine/src/layer.rs:16-26 (fp32, reference layouts)
  ModelWeights       crates/engine/src/full_model.rs:13-17, random 84-90
  CompiledKernels    crates/engine/src/layer.rs:220-275 (compile(cfg))
  forward            crates/engine/src/full_model.rs:345-410 -> ForwardResult.loss
  forward_ws         crates/engine/src/full_model.rs:187-247 -> mean loss
  forward_losses     crates/engine/src/full_model.rs:717-767 -> per-position losses
  Decoder            the single-token loop crates/metal-decode/src/lib.rs:1-8 plans
  backward_ws        crates/engine/src/full_model.rs:250-331 (with forward_ws, one call)
  train_step         crates/engine/src/full_model.rs:661-714

All arithmetic runs on the GPU through the C ABI; this module only moves host
arrays across it.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field, replace
from typing import List, Optional

import numpy as np

from . import hip_bridge as hb


@dataclass
class ModelConfig:
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
    # Constants the reference hard-codes (sdpa_fwd.rs:22, rmsnorm.rs:10,
    # layer.rs:698, full_model.rs:67); 0 selects the reference value.
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    residual_alpha: float = 0.0
    softcap: float = 0.0

    @staticmethod
    def make(dim, hidden, heads, nlayers, seq, vocab, hd=128, kv_heads=None, **kw) -> "ModelConfig":
        kv_heads = heads if kv_heads is None else kv_heads
        return ModelConfig(dim=dim, hidden=hidden, heads=heads, kv_heads=kv_heads, hd=hd, seq=seq,
                           nlayers=nlayers, vocab=vocab, q_dim=heads * hd, kv_dim=kv_heads * hd,
                           gqa_ratio=heads // kv_heads, **kw)

    # -- reference presets (model.rs:21-151) --
    @staticmethod
    def gpt_karpathy():
        return ModelConfig.make(768, 2048, 6, 6, 512, 8192)

    @staticmethod
    def gpt_1024():
        return ModelConfig.make(1024, 2816, 8, 8, 512, 8192)

    @staticmethod
    def target_600m():
        return ModelConfig.make(1536, 4096, 12, 20, 512, 8192)

    @staticmethod
    def target_800m():
        return ModelConfig.make(1792, 4864, 14, 24, 512, 8192)

    @staticmethod
    def target_1b():
        return ModelConfig.make(2048, 5632, 16, 28, 512, 8192)

    @staticmethod
    def target_1_5b():
        return ModelConfig.make(2304, 6144, 18, 32, 512, 8192)

    @staticmethod
    def mha_28l():
        return ModelConfig.make(1024, 3072, 8, 28, 256, 8192)

    # bench_fwd_only_scale.rs:16-27 (hd 128, vocab 8192)
    @staticmethod
    def custom(dim, hidden, heads, nlayers, seq):
        return ModelConfig.make(dim, hidden, heads, nlayers, seq, 8192)

    # -- the measured workloads (vocab 32000) --
    @staticmethod
    def llama_48m():
        return ModelConfig.make(512, 1536, 8, 8, 512, 32000, hd=64)

    @staticmethod
    def llama_600m(seq=512):
        return ModelConfig.make(1536, 4096, 12, 20, seq, 32000)

    @staticmethod
    def llama_5b(seq=512):
        return ModelConfig.make(2560, 6912, 20, 60, seq, 32000)

    @staticmethod
    def llama_7b(seq=512):
        return ModelConfig.make(4096, 11008, 32, 32, seq, 32000)

    def param_count(self) -> int:
        """model.rs:109-114 (counts 4*dim*dim for attention, as the reference does)."""
        per_layer = 4 * self.dim * self.dim + 3 * self.dim * self.hidden
        return self.nlayers * per_layer + self.vocab * self.dim + self.dim * (2 * self.nlayers + 1)

    def alpha(self) -> float:
        return self.residual_alpha or float(np.float32(1.0) / np.sqrt(np.float32(2.0 * self.nlayers)))


@dataclass
class LayerWeights:
    wq: np.ndarray  # [dim*q_dim]
    wk: np.ndarray  # [dim*kv_dim]
    wv: np.ndarray  # [dim*kv_dim]
    wo: np.ndarray  # [q_dim*dim]
    w1: np.ndarray  # [dim*hidden]
    w3: np.ndarray  # [dim*hidden]
    w2: np.ndarray  # [dim*hidden]
    gamma1: np.ndarray
    gamma2: np.ndarray

    @staticmethod
    def random(cfg: ModelConfig) -> "LayerWeights":
        """layer.rs:358-372: Wq/Wk/Wv 1/sqrt(dim), Wo = W2 = 0 (DeepNet), W1/W3 1/sqrt(hidden)."""
        sq = 1.0 / math.sqrt(cfg.dim)
        sf = 1.0 / math.sqrt(cfg.hidden)
        return LayerWeights(
            wq=random_vec(cfg.dim * cfg.q_dim, sq), wk=random_vec(cfg.dim * cfg.kv_dim, sq),
            wv=random_vec(cfg.dim * cfg.kv_dim, sq), wo=np.zeros(cfg.q_dim * cfg.dim, np.float32),
            w1=random_vec(cfg.dim * cfg.hidden, sf), w3=random_vec(cfg.dim * cfg.hidden, sf),
            w2=np.zeros(cfg.dim * cfg.hidden, np.float32),
            gamma1=np.ones(cfg.dim, np.float32), gamma2=np.ones(cfg.dim, np.float32))

    @staticmethod
    def synthetic(cfg: ModelConfig, layer: int, seed: int, std: float = 0.02) -> "LayerWeights":
        """Seeded N(0, std) weights, gammas 1; the same values hb_model_init_synthetic
        writes on the device (tensor ids 16*layer + 0..6)."""
        b = 16 * layer
        n = hb.synth_normal
        d, q, kv, h = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden
        return LayerWeights(
            wq=n(seed, b + 0, d * q, std), wk=n(seed, b + 1, d * kv, std), wv=n(seed, b + 2, d * kv, std),
            wo=n(seed, b + 3, q * d, std), w1=n(seed, b + 4, d * h, std), w3=n(seed, b + 5, d * h, std),
            w2=n(seed, b + 6, d * h, std), gamma1=np.ones(d, np.float32), gamma2=np.ones(d, np.float32))


@dataclass
class ModelWeights:
    embed: np.ndarray  # [vocab*dim]
    layers: List[LayerWeights]
    gamma_final: np.ndarray
    version: int = 0  # bump after mutating arrays in place to force re-upload

    @staticmethod
    def random(cfg: ModelConfig) -> "ModelWeights":
        """full_model.rs:84-90 (embed scale 0.005, gamma 1)."""
        return ModelWeights(embed=random_vec(cfg.vocab * cfg.dim, 0.005),
                            layers=[LayerWeights.random(cfg) for _ in range(cfg.nlayers)],
                            gamma_final=np.ones(cfg.dim, np.float32))

    @staticmethod
    def synthetic(cfg: ModelConfig, seed: int, std: float = 0.02) -> "ModelWeights":
        return ModelWeights(embed=hb.synth_normal(seed, hb.HB_SYNTH_EMBED_ID, cfg.vocab * cfg.dim, std),
                            layers=[LayerWeights.synthetic(cfg, l, seed, std) for l in range(cfg.nlayers)],
                            gamma_final=np.ones(cfg.dim, np.float32))


_LCG_A = np.uint64(6364136223846793005)
_LCG_C = np.uint64(1442695040888963407)


def random_vec(n: int, scale: float) -> np.ndarray:
    """layer.rs:404-413: seed = 42 + n; seed = seed*A + C (wrapping); r = (seed>>32)/u32::MAX*2-1.

    Vectorised with LCG jump-ahead: block k+1 = A^m * block k + C_m elementwise.
    """
    if n == 0:
        return np.zeros(0, np.float32)
    m = min(n, 4096)
    seeds = np.empty(m, np.uint64)
    s = np.uint64(42 + n)
    with np.errstate(over="ignore"):
        for i in range(m):
            s = s * _LCG_A + _LCG_C
            seeds[i] = s
        # jump of m steps: A_m = A^m, C_m = C*(A^(m-1) + ... + 1)
        am, cm = np.uint64(1), np.uint64(0)
        for _ in range(m):
            am, cm = am * _LCG_A, cm * _LCG_A + _LCG_C
        out = np.empty(n, np.uint64)
        blk = seeds
        for start in range(0, n, m):
            take = min(m, n - start)
            out[start:start + take] = blk[:take]
            blk = blk * am + cm
    hi = (out >> np.uint64(32)).astype(np.float32)
    r = (hi / np.float32(4294967295.0)) * np.float32(2.0) - np.float32(1.0)
    return (r * np.float32(scale)).astype(np.float32)


class CompiledKernels:
    """layer.rs:239-274 analogue: a device context + model for one config.

    compile() validates the config and allocates device weights; weights are
    uploaded on the first forward that sees a ModelWeights object (and again
    only when a different object or version is passed).
    """

    def __init__(self, cfg: ModelConfig, device: int = 0):
        self.cfg = cfg
        self.ctx = hb.Context(device)
        self.model = hb.Model(self.ctx, cfg)
        self._uploaded = None

    @staticmethod
    def compile(cfg: ModelConfig, device: int = 0) -> "CompiledKernels":
        return CompiledKernels(cfg, device)

    def ensure_weights(self, weights: Optional[ModelWeights]) -> None:
        if weights is None:
            if self._uploaded is None:
                raise RuntimeError("no weights uploaded")
            return
        key = (id(weights), weights.version)
        if self._uploaded == key:
            return
        for l, lw in enumerate(weights.layers):
            self.model.upload_layer(l, lw)
        self.model.upload_embed(weights.embed, weights.gamma_final)
        self._uploaded = key

    def init_synthetic(self, seed: int, std: float = 0.02) -> None:
        """Device-side seeded weights (no host copy); equals ModelWeights.synthetic."""
        self.model.init_synthetic(seed, std)
        self._uploaded = ("synthetic", seed, std)

    def set_softcap(self, softcap: float) -> None:
        hb.call("hb_model_set_softcap", self.model.handle, float(softcap))


@dataclass
class ForwardLogits:
    """What an inference forward returns (forward_ws's loss with
    forward_losses' per-position losses, full_model.rs:187-247 and 717-767,
    plus the logits the reference keeps in ws.logits, full_model.rs:159,230)."""
    loss: float
    losses: np.ndarray
    logits: Optional[np.ndarray] = None


def _run(cfg, kernels, weights, tokens, targets, softcap, want_logits, batch=1):
    kernels.ensure_weights(weights)
    kernels.set_softcap(softcap)
    tok = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
    T = tok.size
    if T % batch:
        raise ValueError("token count not divisible by batch")
    S = T // batch
    tgt = None if targets is None else np.ascontiguousarray(targets, dtype=np.uint32).reshape(-1)
    losses = np.empty(T, np.float32) if tgt is not None else None
    logits = np.empty((T, cfg.vocab), np.float32) if want_logits else None
    mean = np.zeros(1, np.float32)
    hb.call("hb_forward", kernels.model.handle, hb.ptr(tok), hb.ptr(tgt), batch, S, hb.ptr(losses),
            hb.ptr(logits), hb.ptr(mean) if tgt is not None else None)
    return float(mean[0]), losses, logits


def forward_logits(cfg: ModelConfig, kernels: CompiledKernels, weights: Optional[ModelWeights], tokens,
                   targets, softcap: float = 0.0, want_logits: bool = True, batch: int = 1) -> ForwardLogits:
    """Inference forward (hb_forward): mean loss, per-position losses and the logits."""
    loss, losses, logits = _run(cfg, kernels, weights, tokens, targets, softcap, want_logits, batch)
    return ForwardLogits(loss=loss, losses=losses, logits=logits)


def forward_timed(cfg: ModelConfig, kernels: CompiledKernels, weights: Optional[ModelWeights], tokens,
                  targets, softcap: float = 0.0, batch: int = 1):
    """forward_timed (layer.rs:850-1015) for the whole model (hb_forward_timed):
    the forward's mean loss and the device time of each of its stages (a dict
    of hb_forward_timings' fields, in ms). The tokens go to device buffers
    first (torch provides them); the timed forward is hb_forward_device's."""
    import torch
    kernels.ensure_weights(weights)
    kernels.set_softcap(softcap)
    tok = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
    if tok.size % batch:
        raise ValueError("token count not divisible by batch")
    S = tok.size // batch
    dt = torch.from_numpy(tok.view(np.int32).copy()).cuda()
    dg = None
    if targets is not None:
        dg = torch.from_numpy(np.ascontiguousarray(targets, dtype=np.uint32).reshape(-1).view(np.int32).copy()).cuda()
    dm = torch.zeros(1, device="cuda")
    torch.cuda.synchronize()
    t = kernels.model.forward_timed(dt.data_ptr(), None if dg is None else dg.data_ptr(), batch, S, None,
                                    dm.data_ptr() if dg is not None else None)
    return float(dm.cpu()[0]), t


@dataclass
class ForwardCaches:
    """ForwardResult.caches (full_model.rs:75; layer.rs ForwardCache per layer):
    every layer's activations, kept on the device by the training forward for
    one backward of the same model. Only handles live here."""
    kernels: "CompiledKernels"
    batch: int
    seq: int
    softcap: float = 0.0
    tokens: Optional[np.ndarray] = None


@dataclass
class ForwardResult:
    """full_model.rs:73-81: everything backward needs from forward. The
    arrays are the reference's layouts for one sequence (dlogits [S*V],
    x_final / x_prenorm [dim*S] channel-first, rms_inv_final [S],
    logits_capped [S*V] or empty without softcap); with batch > 1 the
    sequences follow one another."""
    loss: float
    caches: ForwardCaches
    dlogits: np.ndarray
    x_final: np.ndarray
    x_prenorm: np.ndarray
    rms_inv_final: np.ndarray
    logits_capped: np.ndarray


def forward(cfg: ModelConfig, kernels: CompiledKernels, weights: Optional[ModelWeights], tokens,
            targets, softcap: float = 0.0, batch: int = 1) -> ForwardResult:
    """full_model.rs:345-410 (hb_train_forward): embedding, layers, final norm,
    logits, softcap, cross-entropy with its gradient; the per-layer caches stay
    on the device for backward()."""
    kernels.ensure_weights(weights)
    kernels.set_softcap(softcap)
    tok = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
    if tok.size % batch:
        raise ValueError("token count not divisible by batch")
    S = tok.size // batch
    views = ["dlogits", "x_final", "x_prenorm", "rms_inv_final"] + (["logits_capped"] if softcap > 0 else [])
    loss, _, v = kernels.model.train_forward(tok, targets, batch, S, views)
    flat = (lambda a: a.reshape(-1)) if batch == 1 else (lambda a: a)
    caches = ForwardCaches(kernels, batch, S, float(softcap), tok.copy())
    return ForwardResult(loss=loss, caches=caches, dlogits=v["dlogits"],
                         x_final=flat(v["x_final"]), x_prenorm=flat(v["x_prenorm"]),
                         rms_inv_final=v["rms_inv_final"],
                         logits_capped=v.get("logits_capped", np.zeros(0, np.float32)))


def backward(cfg: ModelConfig, kernels: CompiledKernels, weights: Optional[ModelWeights],
             fwd: ForwardResult, tokens, softcap: float, loss_scale: float, grads: "ModelOptState",
             ws=None) -> None:
    """full_model.rs:414-483 from fwd.caches (hb_train_backward): the
    gradients of loss_scale * mean CE are ADDED to grads (the device gradient
    arena of a ModelOptState). `tokens` and `softcap` must be the forward's
    (its activations, capped logits included, stay on the device with the
    caches): anything else raises ValueError before the caches are used;
    `ws` is accepted for the reference's signature, the workspace lives on
    the device."""
    if fwd.caches.kernels is not kernels or grads.kernels is not kernels:
        raise ValueError("fwd and grads must belong to these kernels")
    if float(softcap) != fwd.caches.softcap:
        raise ValueError(f"softcap {softcap} differs from the forward's {fwd.caches.softcap}")
    tok = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
    if fwd.caches.tokens is not None and not np.array_equal(tok, fwd.caches.tokens):
        raise ValueError("tokens differ from the forward's")
    kernels.ensure_weights(weights)
    grads.opt.backward(loss_scale)


def forward_ws(cfg: ModelConfig, kernels: CompiledKernels, weights: Optional[ModelWeights], tokens,
               targets, softcap: float = 0.0, batch: int = 1) -> float:
    return _run(cfg, kernels, weights, tokens, targets, softcap, False, batch)[0]


def forward_losses(cfg: ModelConfig, kernels: CompiledKernels, weights: Optional[ModelWeights],
                   tokens, targets, softcap: float = 0.0, batch: int = 1) -> np.ndarray:
    return _run(cfg, kernels, weights, tokens, targets, softcap, False, batch)[1]


class Decoder:
    """Greedy single-token decode over a preallocated fp16 KV cache."""

    def __init__(self, kernels: CompiledKernels, batch: int, ctx_max: int):
        self.kernels = kernels
        self.cfg = kernels.cfg
        self.kv = hb.KVCache(kernels.model, batch, ctx_max)
        self.batch = batch

    def prefill(self, tokens) -> tuple:
        tok = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        S = tok.size // self.batch
        logits = np.empty((self.batch, self.cfg.vocab), np.float32)
        nxt = np.empty(self.batch, np.uint32)
        hb.call("hb_prefill", self.kernels.model.handle, self.kv.handle, hb.ptr(tok), S,
                hb.ptr(logits), hb.ptr(nxt))
        return logits, nxt

    def step(self, tokens) -> tuple:
        tok = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        logits = np.empty((self.batch, self.cfg.vocab), np.float32)
        nxt = np.empty(self.batch, np.uint32)
        hb.call("hb_decode_step", self.kernels.model.handle, self.kv.handle, hb.ptr(tok),
                hb.ptr(logits), hb.ptr(nxt))
        return logits, nxt

    def greedy(self, first, nsteps: int) -> np.ndarray:
        f = np.ascontiguousarray(first, dtype=np.uint32).reshape(-1)
        out = np.empty((nsteps, self.batch), np.uint32)
        hb.call("hb_decode_greedy", self.kernels.model.handle, self.kv.handle, hb.ptr(f), nsteps,
                hb.ptr(out))
        return out

    def length(self) -> int:
        return self.kv.length()


# ---------------------------------------------------------------------------
# optimizer (full_model.rs:33-70, 334-342, 487-641, 697-711)
# ---------------------------------------------------------------------------
@dataclass
class TrainConfig:
    """full_model.rs:33-70 with its defaults (53-70)."""
    max_lr: float = 3e-4
    min_lr_frac: float = 0.1
    warmup_steps: int = 100
    total_steps: int = 10000
    beta1: float = 0.9
    beta2: float = 0.95
    eps: float = 1e-8
    weight_decay: float = 0.1
    matrix_lr_scale: float = 0.05
    embed_lr_scale: float = 5.0
    loss_scale: float = 256.0
    accum_steps: int = 10
    grad_clip: float = 1.0
    softcap: float = 0.0


def learning_rate(step: int, tc: TrainConfig) -> float:
    """full_model.rs:334-342."""
    return hb.learning_rate(tc, step)


@dataclass
class LayerGrads:
    """layer.rs:29-39 (reference layouts, fp32)."""
    dwq: np.ndarray
    dwk: np.ndarray
    dwv: np.ndarray
    dwo: np.ndarray
    dw1: np.ndarray
    dw3: np.ndarray
    dw2: np.ndarray
    dgamma1: np.ndarray
    dgamma2: np.ndarray

    def as_dict(self) -> dict:
        return dict(wq=self.dwq, wk=self.dwk, wv=self.dwv, wo=self.dwo, w1=self.dw1, w3=self.dw3,
                    w2=self.dw2, gamma1=self.dgamma1, gamma2=self.dgamma2)


@dataclass
class ModelGrads:
    """full_model.rs:20-24."""
    dembed: np.ndarray
    layers: List[LayerGrads]
    dgamma_final: np.ndarray


class ModelOptState:
    """ModelOptState (full_model.rs:26-31) on the device, together with the
    gradient arena and an fp32 master copy of the weights the kernels' fp16
    copy is refreshed from (hb_opt). Built from the model's current weights,
    or from fp32 ModelWeights when given."""

    def __init__(self, kernels: CompiledKernels, tc: TrainConfig,
                 weights: Optional[ModelWeights] = None):
        self.kernels, self.tc = kernels, tc
        self.opt = hb.Optimizer(kernels.model, tc)
        if weights is not None:
            for l, lw in enumerate(weights.layers):
                self.opt.upload_layer(l, lw)
            self.opt.upload_embed(weights.embed, weights.gamma_final)
            kernels._uploaded = (id(weights), weights.version)

    def set_grads(self, grads: ModelGrads) -> None:
        for l, lg in enumerate(grads.layers):
            self.opt.upload_grads_layer(l, lg.as_dict())
        self.opt.upload_grads_embed(grads.dembed, grads.dgamma_final)

    def zero_grads(self) -> None:
        self.opt.zero_grads()

    def close(self) -> None:
        self.opt.close()


def grad_norm(opt: ModelOptState) -> float:
    """full_model.rs:600-622."""
    return opt.opt.grad_norm()


def clip_grads(opt: ModelOptState, max_norm: float) -> float:
    """full_model.rs:625-641; returns the norm before clipping."""
    return opt.opt.clip_grads(max_norm)


def update_weights(opt: ModelOptState, t: int, lr: float, grad_scale: float) -> None:
    """full_model.rs:487-592 (weights, grads and moments live on the device)."""
    opt.opt.update_weights(t, lr, grad_scale)


def optimizer_step(opt: ModelOptState, step: int) -> float:
    """The optimizer half of train_step (full_model.rs:697-711); returns the raw
    gradient norm."""
    return opt.opt.step(step)


def backward_ws(cfg: ModelConfig, kernels: CompiledKernels, opt: ModelOptState, tokens, targets,
                softcap: float, loss_scale: float, batch: int = 1) -> float:
    """forward_ws + backward_ws (full_model.rs:187-331) in one device call
    (hb_forward_backward): the gradients of loss_scale * mean CE of each of
    the `batch` sequences are added to opt's gradient arena. Returns the mean
    loss."""
    kernels.set_softcap(softcap)
    seq = len(np.asarray(tokens).reshape(-1)) // batch
    return opt.opt.forward_backward(tokens, targets, batch, seq, loss_scale)


def train_step(cfg: ModelConfig, kernels: CompiledKernels, opt: ModelOptState, data, step: int,
               tc: TrainConfig) -> float:
    """full_model.rs:661-714: zero the gradients, accum_steps microbatches of
    one sequence at the LCG positions of 682, then the clip decision, the
    learning rate and the AdamW update on the device. Returns the mean loss
    of the microbatches."""
    if opt.tc != tc:
        raise ValueError("tc must be the TrainConfig the optimizer state was created with")
    toks = data._t if isinstance(data, TokenData) else np.asarray(data)
    seq = cfg.seq
    max_pos = len(toks) - seq - 1
    opt.zero_grads()
    total = np.float32(0.0)
    for micro in range(tc.accum_steps):
        pos = random_position(step, micro, max_pos)
        window = np.asarray(toks[pos:pos + seq + 1], dtype=np.uint32)
        total = np.float32(total + np.float32(
            backward_ws(cfg, kernels, opt, window[:-1], window[1:], tc.softcap, tc.loss_scale)))
    opt.opt.step(step, want_norm=False)
    return float(total / np.float32(tc.accum_steps))


# ---------------------------------------------------------------------------
# checkpoints (bin/train.rs:165-202)
# ---------------------------------------------------------------------------
def save_checkpoint(cfg: ModelConfig, kernels: CompiledKernels, opt: Optional[ModelOptState],
                    step: int, directory) -> str:
    """bin/train.rs:165-202: writes <dir>/ckpt_<step:06>.bin (RSTK v1) from the
    optimizer's fp32 master weights, or from the model's fp16 weights when no
    optimizer is given; returns the path."""
    import os
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, f"ckpt_{step:06d}.bin")
    hb.rstk_save(kernels.model, path, step, opt.opt if opt is not None else None)
    return path


def load_checkpoint(path, kernels: CompiledKernels, opt: Optional[ModelOptState] = None) -> int:
    """Load an RSTK checkpoint into the model (and the optimizer's master copy);
    returns its step. The reference has no loader (train.rs only writes)."""
    step = hb.rstk_load(kernels.model, path, opt.opt if opt is not None else None)
    kernels._uploaded = ("rstk", str(path), step)
    return step


# ---------------------------------------------------------------------------
# data path (data.rs) and validation (bin/train.rs:123-163)
# ---------------------------------------------------------------------------
class TokenData:
    """data.rs:11-40: a flat little-endian uint16 token file, memory-mapped."""

    def __init__(self, tokens):
        self._t = tokens
        self._dev = {}

    @staticmethod
    def open(path) -> "TokenData":
        return TokenData(np.memmap(path, dtype="<u2", mode="r"))

    def len(self) -> int:
        return int(self._t.shape[0])

    __len__ = len

    def token(self, pos: int) -> int:
        return int(self._t[pos])

    def tokens(self, start: int, length: int) -> np.ndarray:
        return np.asarray(self._t[start:start + length], dtype=np.uint32)

    def device(self, kernels: CompiledKernels) -> "hb.DeviceTokens":
        """The stream copied once to the kernels' device (cached)."""
        key = id(kernels.ctx)
        if key not in self._dev:
            self._dev[key] = hb.DeviceTokens(kernels.ctx, tokens=np.asarray(self._t))
        return self._dev[key]


class TokenBytes:
    """data.rs:43-58: byte length per token id (int32 little-endian file)."""

    def __init__(self, bytes_per_token):
        self.bytes = np.asarray(bytes_per_token, dtype=np.int32)

    @staticmethod
    def load(path) -> "TokenBytes":
        return TokenBytes(np.fromfile(path, dtype="<i4"))

    def byte_len(self, token_id: int) -> int:
        return int(self.bytes[token_id])


def compute_bpb(losses, targets, token_bytes: TokenBytes):
    """data.rs:61-83 in its fp32 arithmetic: (val_bpb, total_nats, total_bytes)."""
    total_nats = np.float32(0.0)
    total_bytes = 0
    for loss, tok in zip(np.asarray(losses, np.float32), np.asarray(targets)):
        bl = token_bytes.byte_len(int(tok))
        if bl > 0:
            total_nats = np.float32(total_nats + loss)
            total_bytes += bl
    bpb = (np.float32(total_nats / np.float32(np.float32(math.log(2.0)) * np.float32(total_bytes)))
           if total_bytes > 0 else np.float32(0.0))
    return float(bpb), float(total_nats), total_bytes


def random_position(step: int, micro: int, max_pos: int) -> int:
    """data.rs:86-90 (wrapping u64 arithmetic)."""
    mask = (1 << 64) - 1
    seed = ((step * 7919) & mask) + ((micro * 104729) & mask)
    return (seed & mask) % max_pos


def validate(cfg: ModelConfig, kernels: CompiledKernels, weights: Optional[ModelWeights],
             val_data: TokenData, token_bytes: Optional[TokenBytes], steps: int,
             softcap: float = 0.0, batch: int = 1):
    """bin/train.rs:123-163 -> (avg_loss, val_bpb), run on the device: windows
    gathered from the resident token stream, losses and byte counts summed
    there (hb_validate); `batch` windows per forward."""
    kernels.ensure_weights(weights)
    kernels.set_softcap(softcap)
    tb = token_bytes.bytes if token_bytes is not None else None
    avg, bpb, _, _ = hb.validate(kernels.model, val_data.device(kernels), tb, steps, batch)
    return avg, bpb


def validate_host(cfg: ModelConfig, kernels: CompiledKernels, weights: Optional[ModelWeights],
                  val_data: TokenData, token_bytes: Optional[TokenBytes], steps: int,
                  softcap: float = 0.0):
    """The reference's loop as written (train.rs:123-163): one forward_losses call
    per window with host token slices, fp32 sums on the host, compute_bpb."""
    seq = cfg.seq
    total_loss = np.float32(0.0)
    all_losses, all_targets = [], []
    max_pos = val_data.len() - seq - 1
    for vs in range(steps):
        pos = (vs * seq) % max_pos
        inp = val_data.tokens(pos, seq)
        tgt = val_data.tokens(pos + 1, seq)
        losses = forward_losses(cfg, kernels, weights, inp, tgt, softcap)
        total_loss = np.float32(total_loss + np.float32(losses.sum(dtype=np.float32)))
        if token_bytes is not None:
            all_losses.append(losses)
            all_targets.append(tgt)
    avg = float(np.float32(total_loss / np.float32(steps * seq)))
    bpb = 0.0
    if token_bytes is not None:
        bpb = compute_bpb(np.concatenate(all_losses), np.concatenate(all_targets), token_bytes)[0]
    return avg, bpb
