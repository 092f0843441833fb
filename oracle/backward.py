"""fp32 numpy restatement of rustane's backward pass (TEST INFRASTRUCTURE ONLY).

Follows crates/engine/src/layer.rs:1355-1603 (layer backward), the attention
backward graphs of kernels/sdpa_bwd.rs:46-161, the CPU helpers
cpu/rmsnorm.rs:190-236, cpu/cross_entropy.rs:58-96, cpu/embedding.rs:34-44,
layer.rs:1864-1897 (accumulate_dw, rope_backward_inplace) and the model
backward of full_model.rs:412-485, in the reference's channel-first [dim, seq]
layout. Gradients are those of loss_scale * mean cross-entropy (the reference
scales dlogits by loss_scale; train_step divides it out, full_model.rs:697).
Pins: tests/test_backward_oracle.py (torch autograd in float64 on an
independent restatement of the forward, known answers, planted mistakes).
"""
from __future__ import annotations

import numpy as np

from .forward import (Config, ModelW, causal_mask, cross_entropy_batch, embedding_forward,
                      layer_forward, mtrans, rmsnorm_channel_first, rope_backward_cf, rope_table,
                      sgemm_at)

F32 = np.float32
LAYER_TENSORS = ("wq", "wk", "wv", "wo", "w1", "w3", "w2", "gamma1", "gamma2")


def rmsnorm_backward_cf(dy, x, gamma, rms_inv, dim: int, seq: int):
    """cpu/rmsnorm.rs:190-236: x_hat = x r; dgamma[d] = sum_s dy x_hat;
    dot[s] = sum_d dy gamma x_hat / dim; dx = r (dy gamma - x_hat dot).
    Returns (dx [dim*seq], dgamma [dim])."""
    dy = np.asarray(dy, F32).reshape(dim, seq)
    x = np.asarray(x, F32).reshape(dim, seq)
    g = np.asarray(gamma, F32)[:, None]
    r = np.asarray(rms_inv, F32)[None, :]
    x_hat = (x * r).astype(F32)
    dgamma = (dy * x_hat).sum(axis=1, dtype=F32)
    dot = ((dy * g).astype(F32) * x_hat).sum(axis=0, dtype=F32) * (F32(1.0) / F32(dim))
    dx = (r * ((dy * g).astype(F32) - (x_hat * dot[None, :]).astype(F32))).astype(F32)
    return dx.reshape(-1), dgamma.astype(F32)


def cross_entropy_fwd_bwd(logits, targets, vocab: int, inv_seq):
    """cpu/cross_entropy.rs:58-96: per position loss and d = softmax - onehot,
    all scaled by inv_seq. Returns (total loss, dlogits [seq*vocab])."""
    L = np.asarray(logits, F32).reshape(-1, vocab)
    y = np.asarray(targets, np.int64)
    m = L.max(axis=1, keepdims=True)
    sh = (L - m).astype(F32)
    e = np.exp(sh).astype(F32)
    se = e.sum(axis=1, keepdims=True, dtype=F32)
    d = (e * (F32(1.0) / se)).astype(F32)
    d[np.arange(L.shape[0]), y] -= F32(1.0)
    total, _ = cross_entropy_batch(logits, targets, vocab)
    return total, (d * F32(inv_seq)).astype(F32).reshape(-1)


def accumulate_dw(a, a_ch: int, b, b_ch: int, seq: int, dw):
    """layer.rs:1864-1867: dW[a_ch, b_ch] += A[a_ch, seq] B[b_ch, seq]^T (flat result)."""
    return sgemm_at(a, a_ch, seq, b, b_ch, dw).reshape(-1)


def _dyn_matmul_t(acts_cf, w, ic: int, oc: int, seq: int):
    """out[oc, s] = sum_ic acts[ic, s] W[ic, oc] (kernels/dyn_matmul.rs form)."""
    a = np.asarray(acts_cf, F32).reshape(ic, seq)
    return (a.T @ np.asarray(w, F32).reshape(ic, oc)).T.astype(F32)


def sdpa_backward(cfg: Config, q_rope, k_rope, v, da, seq: int):
    """kernels/sdpa_bwd.rs: bwd1 (46-105) recomputes probs = softmax(QK^T scale +
    mask) and gives dV = probs^T da, dp = da V^T; bwd2 (108-161) gives
    ds = probs (dp - sum(probs dp)) scale, dQ = ds K, dK = ds^T Q. Channel-first
    [H*hd, seq] in and out. GQA (not in the reference, which tiles K/V for MHA):
    dK/dV of a kv head sum its query heads' contributions."""
    H, KVH, hd = cfg.heads, cfg.kv_heads, cfg.hd
    rep = H // KVH
    scale = F32(1.0) / np.sqrt(F32(hd))
    q = np.asarray(q_rope, F32).reshape(H, hd, seq).transpose(0, 2, 1)
    k = np.repeat(np.asarray(k_rope, F32).reshape(KVH, hd, seq).transpose(0, 2, 1), rep, axis=0)
    vv = np.repeat(np.asarray(v, F32).reshape(KVH, hd, seq).transpose(0, 2, 1), rep, axis=0)
    d = np.asarray(da, F32).reshape(H, hd, seq).transpose(0, 2, 1)
    sc = ((q @ k.transpose(0, 2, 1)).astype(F32) * scale + causal_mask(seq)[None]).astype(F32)
    m = sc.max(axis=-1, keepdims=True)
    e = np.exp((sc - m).astype(F32)).astype(F32)
    probs = (e / e.sum(axis=-1, keepdims=True, dtype=F32)).astype(F32)
    dv = (probs.transpose(0, 2, 1) @ d).astype(F32)            # [H, seq, hd]
    dp = (d @ vv.transpose(0, 2, 1)).astype(F32)               # [H, seq, seq]
    spdp = (probs * dp).astype(F32).sum(axis=-1, keepdims=True, dtype=F32)
    ds = ((probs * (dp - spdp).astype(F32)).astype(F32) * scale).astype(F32)
    dq = (ds @ k).astype(F32)
    dk = (ds.transpose(0, 2, 1) @ q).astype(F32)
    if rep > 1:
        dk = dk.reshape(KVH, rep, seq, hd).sum(axis=1, dtype=F32)
        dv = dv.reshape(KVH, rep, seq, hd).sum(axis=1, dtype=F32)
    cf = lambda t, nh: np.ascontiguousarray(t.transpose(0, 2, 1)).reshape(nh * hd, seq)
    return cf(dq, H), cf(dk, KVH), cf(dv, KVH)


def layer_backward(cfg: Config, lw, taps: dict, x_in, dy, seq: int):
    """layer.rs:1355-1603 for one layer. taps: the forward's intermediates
    (oracle.forward.layer_forward); x_in: the layer input [dim*seq]; dy: the
    gradient of its output. Returns (dx [dim*seq], grads dict per LAYER_TENSORS)."""
    d, q, kv, h = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden
    alpha = cfg.alpha()
    dy = np.asarray(dy, F32).reshape(-1)
    g = {k: np.zeros_like(np.asarray(getattr(lw, k), F32)) for k in LAYER_TENSORS}
    # 1-2: dffn = alpha dy; dsilu_raw = W2^T dffn (ffnBwdW2t)
    dffn = (dy * alpha).astype(F32)
    dsilu = _dyn_matmul_t(dffn, lw.w2, d, h, seq)
    # 3: SiLU derivative
    h1 = np.asarray(taps["h1"], F32).reshape(h, seq)
    h3 = np.asarray(taps["h3"], F32).reshape(h, seq)
    with np.errstate(over="ignore"):
        sig = (F32(1.0) / (F32(1.0) + np.exp(-h1))).astype(F32)
    silu = (h1 * sig).astype(F32)
    dsilu_dx = (sig * (F32(1.0) + (h1 * (F32(1.0) - sig)).astype(F32))).astype(F32)
    dh3 = (dsilu * silu).astype(F32)
    dh1 = ((dsilu * h3).astype(F32) * dsilu_dx).astype(F32)
    # 4-5: dx_ffn = W1 dh1 + W3 dh3 (ffnBwdW13t); dW3 += x2norm dh3^T
    w1t = mtrans(lw.w1, d, h)
    w3t = mtrans(lw.w3, d, h)
    dx_ffn = (_dyn_matmul_t(dh1, w1t, h, d, seq) + _dyn_matmul_t(dh3, w3t, h, d, seq)).astype(F32)
    g["w3"] = accumulate_dw(taps["x2norm"], d, dh3, h, seq, g["w3"])
    # 6: RMSNorm2 backward, + dy (FFN residual)
    dx2, dg2 = rmsnorm_backward_cf(dx_ffn, taps["x2"], lw.gamma2, taps["rms_inv2"], d, seq)
    g["gamma2"] = (g["gamma2"] + dg2).astype(F32)
    dx2 = (dx2 + dy).astype(F32)
    # 7-8: dx2s = alpha dx2; da = Wo dx2s (wotBwd)
    dx2s = (dx2 * alpha).astype(F32)
    da = _dyn_matmul_t(dx2s, mtrans(lw.wo, q, d), d, q, seq)
    # 9: dWo += attn dx2s^T; dW2 += dffn gate^T
    g["wo"] = accumulate_dw(taps["attn"], q, dx2s, d, seq, g["wo"])
    g["w2"] = accumulate_dw(dffn, d, taps["gate"], h, seq, g["w2"])
    # 10-11: attention backward
    dq, dk, dv = sdpa_backward(cfg, taps["q_rope"], taps["k_rope"], taps["v"], da, seq)
    g["w1"] = accumulate_dw(taps["x2norm"], d, dh1, h, seq, g["w1"])
    # 12: RoPE backward (the RopeTable of layer.rs:203-216)
    dq = rope_backward_cf(dq, cfg.heads, cfg.hd, seq, cfg.rope_theta)
    dk = rope_backward_cf(dk, cfg.kv_heads, cfg.hd, seq, cfg.rope_theta)
    # 13: dWq/dWk/dWv; dx_attn = Wq dq; dx_kv = Wk dk + Wv dv
    g["wq"] = accumulate_dw(taps["xnorm"], d, dq, q, seq, g["wq"])
    g["wk"] = accumulate_dw(taps["xnorm"], d, dk, kv, seq, g["wk"])
    g["wv"] = accumulate_dw(taps["xnorm"], d, dv, kv, seq, g["wv"])
    dx_attn = _dyn_matmul_t(dq, mtrans(lw.wq, d, q), q, d, seq)
    dx_kv = (_dyn_matmul_t(dk, mtrans(lw.wk, d, kv), kv, d, seq)
             + _dyn_matmul_t(dv, mtrans(lw.wv, d, kv), kv, d, seq)).astype(F32)
    # 14-17: merge, RMSNorm1 backward, + dx2 (attention residual)
    dx_merged = (dx_attn + dx_kv).astype(F32)
    dx1, dg1 = rmsnorm_backward_cf(dx_merged, x_in, lw.gamma1, taps["rms_inv1"], d, seq)
    g["gamma1"] = (g["gamma1"] + dg1).astype(F32)
    return (dx1 + dx2.reshape(-1)).astype(F32), g


def model_forward_backward(cfg: Config, w: ModelW, tokens, targets, softcap: float = 0.0,
                           loss_scale: float = 1.0):
    """forward_ws (full_model.rs:187-247) + backward (412-485) for one sequence.
    Returns (mean loss, grads {"embed", "gamma_final", "layers": [...]})."""
    d, V = cfg.dim, cfg.vocab
    seq = len(tokens)
    x = mtrans(embedding_forward(w.embed, d, tokens), seq, d)
    rope = rope_table(seq, cfg.hd, cfg.rope_theta)
    inputs, taps = [], []
    for l in range(cfg.nlayers):
        inputs.append(x)
        x, t = layer_forward(cfg, w.layers[l], x, seq, rope)
        taps.append(t)
    x_prenorm = x
    xf, rinv_f = rmsnorm_channel_first(x_prenorm, w.gamma_final, d, seq, cfg.norm_eps)
    logits = sgemm_at(mtrans(xf, d, seq), seq, d, w.embed, V, np.zeros(seq * V, F32)).reshape(-1)
    t_cap = None
    if softcap > 0.0:
        t_cap = np.tanh((logits * (F32(1.0) / F32(softcap))).astype(F32)).astype(F32)
        logits = (t_cap * F32(softcap)).astype(F32)
    total, dlogits = cross_entropy_fwd_bwd(logits, targets, V, F32(1.0) / F32(seq))
    # full_model.rs:429-440: dl = dlogits * loss_scale (* (1 - t^2) with softcap)
    dl = (dlogits * F32(loss_scale)).astype(F32)
    if t_cap is not None:
        dl = (dl * (F32(1.0) - (t_cap * t_cap).astype(F32))).astype(F32)
    dl = dl.reshape(seq, V)
    grads = {"embed": np.zeros(V * d, F32), "gamma_final": np.zeros(d, F32), "layers": []}
    xf2 = np.asarray(xf, F32).reshape(d, seq)
    # 442-453: dembed += dl^T x_final^T; dx_final = embed^T dl^T
    grads["embed"] = (grads["embed"].reshape(V, d) + (dl.T @ xf2.T).astype(F32)).astype(F32).reshape(-1)
    dx_final = (np.asarray(w.embed, F32).reshape(V, d).T @ dl.T).astype(F32).reshape(-1)
    # 468-471: final RMSNorm backward
    dy, dgf = rmsnorm_backward_cf(dx_final, x_prenorm, w.gamma_final, rinv_f, d, seq)
    grads["gamma_final"] = (grads["gamma_final"] + dgf).astype(F32)
    layer_grads = [None] * cfg.nlayers
    for l in range(cfg.nlayers - 1, -1, -1):
        dy, layer_grads[l] = layer_backward(cfg, w.layers[l], taps[l], inputs[l], dy, seq)
    grads["layers"] = layer_grads
    # 482-483: embedding backward, channel-first scatter-add
    e = grads["embed"].reshape(V, d)
    dyc = dy.reshape(d, seq)
    for s, tok in enumerate(np.asarray(tokens, np.int64)):
        e[tok] += dyc[:, s]
    return F32(total / F32(seq)), grads
