"""numpy restatement of rustane's optimizer step (TEST INFRASTRUCTURE ONLY).

AdamW (crates/engine/src/cpu/adam.rs), the global gradient norm, clipping, the
learning-rate schedule and the per-group update of full_model.rs. Every value
is fp32 and every operation is rounded to fp32 in the reference's evaluation
order, so the device kernel (which disables fused multiply-adds) can be
compared bit for bit. Pins: tests/test_optimizer_oracle.py.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

F32 = np.float32


@dataclass
class TrainConfig:
    """TrainConfig with the defaults of full_model.rs:53-70."""
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


def powi_f32(a, b: int) -> np.float32:
    """f32::powi as cpu/adam.rs:113-114 uses it: llvm.powi.f32, which lowers to
    compiler-rt's __powisf2 -- exponentiation by squaring in fp32."""
    a = F32(a)
    recip = b < 0
    r = F32(1.0)
    while True:
        if b & 1:
            r = F32(r * a)
        b = int(b / 2)  # truncating division, as in C
        if b == 0:
            break
        a = F32(a * a)
    return F32(F32(1.0) / r) if recip else r


def bias_corrections(beta1, beta2, t: int):
    """cpu/adam.rs:113-114: bc = 1 / (1 - beta^t)."""
    bc1 = F32(F32(1.0) / F32(F32(1.0) - powi_f32(beta1, t)))
    bc2 = F32(F32(1.0) / F32(F32(1.0) - powi_f32(beta2, t)))
    return bc1, bc2


def step_fused(param, grad, m, v, t: int, lr, beta1, beta2, eps, weight_decay, grad_scale):
    """cpu/adam.rs:95-132 (and the Metal shader metal_adam.rs:13-38): in place on
    param, m, v (fp32 numpy arrays), one pass:
      g = grad * grad_scale; m = b1 m + (1-b1) g; v = b2 v + (1-b2) g g;
      update = (m bc1) / (sqrt(v bc2) + eps); param -= lr (update + wd param)."""
    assert t > 0
    b1, b2 = F32(beta1), F32(beta2)
    bc1, bc2 = bias_corrections(b1, b2, t)
    omb1, omb2 = F32(F32(1.0) - b1), F32(F32(1.0) - b2)
    g = (np.asarray(grad, F32) * F32(grad_scale)).astype(F32)
    mi = (b1 * m).astype(F32) + (omb1 * g).astype(F32)
    vi = (b2 * v).astype(F32) + ((omb2 * g).astype(F32) * g).astype(F32)
    m[...] = mi
    v[...] = vi
    m_hat = (mi * bc1).astype(F32)
    v_hat = (vi * bc2).astype(F32)
    update = (m_hat / (np.sqrt(v_hat) + F32(eps)).astype(F32)).astype(F32)
    decay = (F32(weight_decay) * param).astype(F32)
    param[...] = (param - (F32(lr) * (update + decay).astype(F32)).astype(F32)).astype(F32)


def step(param, grad, m, v, t: int, lr, beta1, beta2, eps, weight_decay):
    """cpu/adam.rs:37-85, the multi-pass vDSP form of the same step (no grad
    scale): m = grad*(1-b1) + b1*m, v = (grad*grad)*(1-b2) + b2*v, then the
    bias-corrected update."""
    b1, b2 = F32(beta1), F32(beta2)
    tmp = (b1 * m).astype(F32)
    m[...] = ((np.asarray(grad, F32) * F32(F32(1.0) - b1)).astype(F32) + tmp).astype(F32)
    tmp = (np.asarray(grad, F32) * np.asarray(grad, F32)).astype(F32)
    tmp2 = (b2 * v).astype(F32)
    v[...] = ((tmp * F32(F32(1.0) - b2)).astype(F32) + tmp2).astype(F32)
    bc1, bc2 = bias_corrections(b1, b2, t)
    mh = (m * bc1).astype(F32)
    vh = (v * bc2).astype(F32)
    update = (mh / (np.sqrt(vh) + F32(eps)).astype(F32)).astype(F32)
    param[...] = (param - (F32(lr) * (update + (F32(weight_decay) * param).astype(F32))
                           .astype(F32)).astype(F32)).astype(F32)


def learning_rate(step: int, tc: TrainConfig) -> np.float32:
    """full_model.rs:334-342: linear warmup, then cosine decay to max_lr*min_lr_frac (fp32)."""
    max_lr = F32(tc.max_lr)
    if step < tc.warmup_steps:
        return F32(F32(max_lr * F32(step + 1)) / F32(tc.warmup_steps))
    decay = F32(F32(step - tc.warmup_steps) / F32(tc.total_steps - tc.warmup_steps))
    min_lr = F32(max_lr * F32(tc.min_lr_frac))
    c = F32(np.cos(F32(F32(math.pi) * decay)))
    return F32(min_lr + F32(F32(F32(0.5) * F32(F32(1.0) + c)) * F32(max_lr - min_lr)))


LAYER_TENSORS = ("wq", "wk", "wv", "wo", "w1", "w3", "w2", "gamma1", "gamma2")
MATRICES = ("wq", "wk", "wv", "wo", "w1", "w3", "w2")


def grad_norm(grads) -> np.float32:
    """full_model.rs:600-622: sqrt of the sum of squares of every gradient
    (dembed, dgamma_final and each layer's nine tensors), accumulated here in
    fp64 and rounded once."""
    s = np.float64(0.0)
    s += np.sum(np.square(grads["embed"].astype(np.float64)))
    s += np.sum(np.square(grads["gamma_final"].astype(np.float64)))
    for lg in grads["layers"]:
        for k in LAYER_TENSORS:
            s += np.sum(np.square(lg[k].astype(np.float64)))
    return F32(math.sqrt(s))


def clip_grads(grads, max_norm) -> np.float32:
    """full_model.rs:625-641: scale every gradient by max_norm/norm when norm > max_norm."""
    norm = grad_norm(grads)
    if norm > F32(max_norm):
        scale = F32(F32(max_norm) / norm)
        grads["embed"] *= scale
        grads["gamma_final"] *= scale
        for lg in grads["layers"]:
            for k in LAYER_TENSORS:
                lg[k] *= scale
    return norm


def combined_scale(raw_norm, tc: TrainConfig) -> np.float32:
    """full_model.rs:697-705: descale by 1/(accum_steps*loss_scale), or clip."""
    gsc = F32(F32(1.0) / F32(F32(tc.accum_steps) * F32(tc.loss_scale)))
    scaled = F32(F32(raw_norm) * gsc)
    return F32(F32(tc.grad_clip) / F32(raw_norm)) if scaled > F32(tc.grad_clip) else gsc


def update_weights(weights, grads, opt, t: int, lr, tc: TrainConfig, grad_scale):
    """full_model.rs:487-592 (update_layer 569-592): matrices at lr*matrix_lr_scale
    with weight decay, the embedding at lr*embed_lr_scale and the gammas at lr,
    both without. weights / grads / opt['m'] / opt['v'] are dicts
    {"embed", "gamma_final", "layers": [dict per LAYER_TENSORS]} of fp32 arrays,
    updated in place."""
    lr = F32(lr)
    matrix_lr = F32(lr * F32(tc.matrix_lr_scale))
    embed_lr = F32(lr * F32(tc.embed_lr_scale))
    args = (t,)
    hp = (tc.beta1, tc.beta2, tc.eps)
    step_fused(weights["embed"], grads["embed"], opt["m"]["embed"], opt["v"]["embed"], *args,
               embed_lr, *hp, 0.0, grad_scale)
    step_fused(weights["gamma_final"], grads["gamma_final"], opt["m"]["gamma_final"],
               opt["v"]["gamma_final"], *args, lr, *hp, 0.0, grad_scale)
    for l, lw in enumerate(weights["layers"]):
        lg, lm, lv = grads["layers"][l], opt["m"]["layers"][l], opt["v"]["layers"][l]
        for k in MATRICES:
            step_fused(lw[k], lg[k], lm[k], lv[k], *args, matrix_lr, *hp, tc.weight_decay, grad_scale)
        for k in ("gamma1", "gamma2"):
            step_fused(lw[k], lg[k], lm[k], lv[k], *args, lr, *hp, 0.0, grad_scale)


def optimizer_step(weights, grads, opt, step: int, tc: TrainConfig):
    """The optimizer half of train_step (full_model.rs:697-711): norm, combined
    scale, learning_rate(step), update_weights(t = step + 1). Returns the raw norm."""
    raw = grad_norm(grads)
    update_weights(weights, grads, opt, step + 1, learning_rate(step, tc), tc,
                   combined_scale(raw, tc))
    return raw


def zeros_like_state(weights):
    """ModelOptState::new / ModelGrads::zeros: zero arrays shaped like the weights."""
    return {"embed": np.zeros_like(weights["embed"]),
            "gamma_final": np.zeros_like(weights["gamma_final"]),
            "layers": [{k: np.zeros_like(lw[k]) for k in LAYER_TENSORS} for lw in weights["layers"]]}
