"""fp32 numpy restatement of rustane's forward path (TEST INFRASTRUCTURE ONLY).

Every function follows the reference file:line named in its docstring. Layouts
follow the reference: activations are channel-first [dim, seq] (the IOSurface
layout, crates/engine/src/layer.rs:42-85), weights are the LayerWeights /
ModelWeights fp32 arrays (layer.rs:16-26, full_model.rs:13-17).

Where the reference delegates to Accelerate (cblas_sgemm, vDSP) the oracle uses
numpy's BLAS (`@`), as the portable stand-in; where the reference runs a graph
on the ANE in fp16 the oracle computes the same graph in fp32.

Pinning status (tests/test_oracle.py): every function below has at least one
known-answer, closed-form, brute-force or independent-implementation check.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import numpy as np

F32 = np.float32
EPS = F32(1e-5)  # cpu/rmsnorm.rs:10
MASK_NEG = F32(-65504.0)  # kernels/sdpa_fwd.rs:35-46 (fp16 -inf)

__all__ = [
    "Config", "LayerW", "ModelW", "embedding_forward", "mtrans", "rmsnorm_forward",
    "rmsnorm_channel_first", "rope_table", "rope_apply_cf", "rope_backward_cf", "causal_mask",
    "sdpa_fwd", "dyn_matmul", "vsma", "silu_gate", "ffn_fused", "layer_forward",
    "cross_entropy_forward", "cross_entropy_batch", "model_forward", "forward_batch",
    "DecodeOracle", "sgemm_at", "softcap_forward",
]


@dataclass
class Config:
    """ModelConfig (crates/engine/src/model.rs:5-17) + the constants the reference fixes."""
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
    gqa_ratio: int = 1
    rope_theta: float = 10000.0
    norm_eps: float = 1e-5
    residual_alpha: float = 0.0
    softcap: float = 0.0

    def alpha(self) -> np.float32:
        """layer.rs:698 / ffn_fused.rs:29: 1 / sqrt(2 * nlayers) in f32."""
        if self.residual_alpha:
            return F32(self.residual_alpha)
        return F32(1.0) / np.sqrt(F32(2.0) * F32(self.nlayers))

    @staticmethod
    def of(cfg) -> "Config":
        return Config(**{k: getattr(cfg, k) for k in Config.__dataclass_fields__})


@dataclass
class LayerW:
    wq: np.ndarray
    wk: np.ndarray
    wv: np.ndarray
    wo: np.ndarray
    w1: np.ndarray
    w3: np.ndarray
    w2: np.ndarray
    gamma1: np.ndarray
    gamma2: np.ndarray


@dataclass
class ModelW:
    embed: np.ndarray
    layers: List[LayerW]
    gamma_final: np.ndarray

    @staticmethod
    def of(w) -> "ModelW":
        return ModelW(embed=np.asarray(w.embed, F32),
                      layers=[LayerW(**{k: np.asarray(getattr(l, k), F32) for k in LayerW.__dataclass_fields__})
                              for l in w.layers],
                      gamma_final=np.asarray(w.gamma_final, F32))


# ---------------------------------------------------------------------------
# CPU ops (crates/engine/src/cpu/*.rs)
# ---------------------------------------------------------------------------

def embedding_forward(table: np.ndarray, dim: int, token_ids: Sequence[int]) -> np.ndarray:
    """cpu/embedding.rs:8-16: out[s*dim .. (s+1)*dim] = table[tok*dim .. (tok+1)*dim]."""
    t = np.asarray(table, F32).reshape(-1, dim)
    ids = np.asarray(token_ids, np.int64)
    return t[ids].reshape(-1).copy()


def mtrans(a: np.ndarray, m: int, n: int) -> np.ndarray:
    """cpu/vdsp.rs:245-251: C[n,m] = A[m,n]^T (flat row-major in and out)."""
    return np.ascontiguousarray(np.asarray(a, F32).reshape(m, n).T).reshape(-1)


def rmsnorm_forward(x: np.ndarray, gamma: np.ndarray):
    """cpu/rmsnorm.rs:15-38 (single vector): rms_inv = 1/sqrt(mean(x^2) + eps); out = x*rms_inv*gamma."""
    x = np.asarray(x, F32)
    g = np.asarray(gamma, F32)
    sq = x * x
    acc = F32(0.0)
    for v in sq:  # vDSP_sve: sequential sum
        acc = F32(acc + v)
    mean_sq = F32(acc / F32(x.size))
    rms_inv = F32(1.0) / np.sqrt(F32(mean_sq + EPS))
    out = (x * rms_inv).astype(F32) * g
    return out.astype(F32), F32(rms_inv)


def rmsnorm_channel_first(x: np.ndarray, gamma: np.ndarray, dim: int, seq: int, eps=EPS):
    """cpu/rmsnorm.rs:149-183 on channel-first [dim, seq]:
    sum_sq[s] accumulated over d in channel order (f32), rms_inv = 1/sqrt(sum_sq*(1/dim) + eps),
    out[d,s] = x[d,s] * rms_inv[s] * gamma[d]."""
    x = np.asarray(x, F32).reshape(dim, seq)
    acc = np.zeros(seq, F32)
    for d in range(dim):
        row = x[d]
        acc += row * row
    inv_dim = F32(1.0) / F32(dim)
    rms_inv = (F32(1.0) / np.sqrt(acc * inv_dim + F32(eps))).astype(F32)
    out = (x * rms_inv[None, :]) * np.asarray(gamma, F32)[:, None]
    return out.astype(F32).reshape(-1), rms_inv


def vsma(a: np.ndarray, scalar, b: np.ndarray) -> np.ndarray:
    """cpu/vdsp.rs:178-181: out = a * scalar + b."""
    return (np.asarray(a, F32) * F32(scalar) + np.asarray(b, F32)).astype(F32)


def silu_gate(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """cpu/silu.rs:37-46: out = gate * (1/(1+exp(-gate))) * up (also the ANE graph
    kernels/ffn_fused.rs:60-62: h1 * sigmoid(h1) * h3)."""
    g = np.asarray(gate, F32)
    with np.errstate(over="ignore"):
        sig = F32(1.0) / (F32(1.0) + np.exp(-g))
    return (g * sig * np.asarray(up, F32)).astype(F32)


def sgemm_at(a: np.ndarray, m: int, k: int, b: np.ndarray, n: int, c: np.ndarray) -> np.ndarray:
    """cpu/vdsp.rs:287-302: C += A @ B^T (beta = 1 accumulates; callers zero C first,
    full_model.rs:229)."""
    A = np.asarray(a, F32).reshape(m, k)
    Bm = np.asarray(b, F32).reshape(n, k)
    c = np.asarray(c, F32).reshape(m, n)
    return (c + A @ Bm.T).astype(F32)


def cross_entropy_forward(logits: np.ndarray, target: int):
    """cpu/cross_entropy.rs:13-38: shifted = x - max; log_sm = shifted - ln(sum(exp(shifted)));
    loss = -log_sm[target]."""
    x = np.asarray(logits, F32)
    if not 0 <= target < x.size:
        raise ValueError("target out of range")
    m = x.max()
    shifted = (x - m).astype(F32)
    sum_exp = np.exp(shifted).astype(F32).sum(dtype=F32)
    log_sm = (shifted - F32(np.log(sum_exp))).astype(F32)
    return F32(-log_sm[target]), log_sm


def cross_entropy_batch(logits: np.ndarray, targets: Sequence[int], vocab: int):
    """cpu/cross_entropy.rs:58-96 (forward part): per position loss = -(shifted[y] - ln(sum_exp));
    returns (total loss, per-position losses)."""
    L = np.asarray(logits, F32).reshape(-1, vocab)
    y = np.asarray(targets, np.int64)
    m = L.max(axis=1, keepdims=True)
    shifted = (L - m).astype(F32)
    sum_exp = np.exp(shifted).astype(F32).sum(axis=1, dtype=F32)
    losses = (-(shifted[np.arange(L.shape[0]), y] - np.log(sum_exp))).astype(F32)
    total = F32(0.0)
    for v in losses:
        total = F32(total + v)
    return total, losses


# ---------------------------------------------------------------------------
# ANE graphs (crates/engine/src/kernels/*.rs), computed in fp32
# ---------------------------------------------------------------------------

def rope_table(seq: int, hd: int, theta: float = 10000.0):
    """kernels/sdpa_fwd.rs:18-33: theta_p,i = p / base^(2i/hd) (f32); cos/sin duplicated over
    the pair (2i, 2i+1); returns [seq, hd] tables."""
    cos = np.zeros((seq, hd), F32)
    sin = np.zeros((seq, hd), F32)
    base = F32(theta)
    for i in range(hd // 2):
        freq_den = np.power(base, F32(2.0) * F32(i) / F32(hd), dtype=F32)
        th = (np.arange(seq, dtype=F32) / freq_den).astype(F32)
        c, s = np.cos(th).astype(F32), np.sin(th).astype(F32)
        cos[:, 2 * i] = c
        cos[:, 2 * i + 1] = c
        sin[:, 2 * i] = s
        sin[:, 2 * i + 1] = s
    return cos, sin


def rope_apply_cf(x_cf: np.ndarray, heads: int, hd: int, seq: int, cos, sin, pos0: int = 0):
    """kernels/sdpa_fwd.rs:105-128 on a channel-first [heads*hd, seq] tensor:
    rot(x) pairs = (-x[2i+1], x[2i]); out = x*cos + rot(x)*sin, i.e.
    out[2i] = x[2i] c - x[2i+1] s, out[2i+1] = x[2i+1] c + x[2i] s. Position of column s
    is pos0 + s."""
    x = np.asarray(x_cf, F32).reshape(heads, hd, seq)
    c = cos[pos0:pos0 + seq].T[None]  # [1, hd, seq]
    s = sin[pos0:pos0 + seq].T[None]
    rot = np.empty_like(x)
    rot[:, 0::2, :] = -x[:, 1::2, :]
    rot[:, 1::2, :] = x[:, 0::2, :]
    return (x * c + rot * s).astype(F32).reshape(heads * hd, seq)


def rope_backward_cf(dx_cf: np.ndarray, heads: int, hd: int, seq: int, theta: float = 10000.0):
    """layer.rs:1880-1897 with the RopeTable of layer.rs:203-216 (freq = 1/base^(2i/hd),
    theta = p*freq): the inverse rotation d0' = c d0 + s d1, d1' = -s d0 + c d1."""
    dx = np.asarray(dx_cf, F32).reshape(heads, hd, seq).copy()
    for i in range(hd // 2):
        freq = F32(1.0) / np.power(F32(theta), F32(2.0) * F32(i) / F32(hd), dtype=F32)
        th = (np.arange(seq, dtype=F32) * freq).astype(F32)
        c, s = np.cos(th).astype(F32), np.sin(th).astype(F32)
        d0 = dx[:, 2 * i, :].copy()
        d1 = dx[:, 2 * i + 1, :].copy()
        dx[:, 2 * i, :] = c * d0 + s * d1
        dx[:, 2 * i + 1, :] = -s * d0 + c * d1
    return dx.reshape(heads * hd, seq)


def causal_mask(seq: int) -> np.ndarray:
    """kernels/sdpa_fwd.rs:36-46: 0 where t2 <= t, -65504 where t2 > t."""
    m = np.zeros((seq, seq), F32)
    m[np.triu_indices(seq, 1)] = MASK_NEG
    return m


def _softmax_last(x: np.ndarray) -> np.ndarray:
    m = x.max(axis=-1, keepdims=True)
    e = np.exp((x - m).astype(F32)).astype(F32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=F32)).astype(F32)


def sdpa_fwd(cfg: Config, xnorm_cf: np.ndarray, wq, wk, wv, seq: int, rope=None):
    """kernels/sdpa_fwd.rs:49-161: Q/K/V = xnorm^T @ W (70-90); heads j = h*hd+e (93-98);
    interleaved RoPE on Q, K (105-128); scores = Q K^T * (1/sqrt(hd)) + mask (132-140);
    softmax over keys (142); attn = P V (145); output channel-first [q_dim, seq] (148-149).
    GQA: query head h reads kv head h // gqa_ratio (MHA when gqa_ratio = 1).
    Returns dict(attn, q_rope, k_rope, v) channel-first."""
    d, q, kv, H, KVH, hd = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.heads, cfg.kv_heads, cfg.hd
    xnt = np.asarray(xnorm_cf, F32).reshape(d, seq).T  # [seq, dim]
    Qf = (xnt @ np.asarray(wq, F32).reshape(d, q)).T  # [q, seq]
    Kf = (xnt @ np.asarray(wk, F32).reshape(d, kv)).T
    Vf = (xnt @ np.asarray(wv, F32).reshape(d, kv)).T
    cos, sin = rope if rope is not None else rope_table(seq, hd, cfg.rope_theta)
    Qr = rope_apply_cf(Qf, H, hd, seq, cos, sin)
    Kr = rope_apply_cf(Kf, KVH, hd, seq, cos, sin)
    q4 = Qr.reshape(H, hd, seq).transpose(0, 2, 1)  # [H, seq, hd]
    k4 = Kr.reshape(KVH, hd, seq).transpose(0, 2, 1)
    v4 = np.ascontiguousarray(Vf).reshape(KVH, hd, seq).transpose(0, 2, 1)
    rep = H // KVH
    k4 = np.repeat(k4, rep, axis=0)
    v4 = np.repeat(v4, rep, axis=0)
    scale = F32(1.0) / np.sqrt(F32(hd))
    sc = (q4 @ k4.transpose(0, 2, 1)).astype(F32) * scale + causal_mask(seq)[None]
    p = _softmax_last(sc.astype(F32))
    a4 = (p @ v4).astype(F32)  # [H, seq, hd]
    attn = a4.transpose(0, 2, 1).reshape(q, seq)
    return {"attn": np.ascontiguousarray(attn, F32), "q_rope": Qr, "k_rope": Kr,
            "v": np.ascontiguousarray(Vf, F32)}


def dyn_matmul(acts_cf: np.ndarray, w: np.ndarray, ic: int, oc: int, seq: int) -> np.ndarray:
    """kernels/dyn_matmul.rs:15-46: out[oc, seq] = (acts^T @ W)^T, W [ic, oc]."""
    a = np.asarray(acts_cf, F32).reshape(ic, seq)
    return (a.T @ np.asarray(w, F32).reshape(ic, oc)).T.astype(F32)


def ffn_fused(cfg: Config, x2norm_cf, x2_cf, w1, w3, w2, seq: int):
    """kernels/ffn_fused.rs:22-83: h1 = xn@W1, h3 = xn@W3 (43-57), gate = silu(h1)*h3
    (60-62), ffn = gate @ W2^T with W2 stored [dim, hidden] (65-72),
    x_next = x2 + alpha*ffn (74-77). Returns dict(x_next, h1, h3, gate) channel-first."""
    d, h = cfg.dim, cfg.hidden
    xnt = np.asarray(x2norm_cf, F32).reshape(d, seq).T
    h1 = (xnt @ np.asarray(w1, F32).reshape(d, h)).T  # [h, seq]
    h3 = (xnt @ np.asarray(w3, F32).reshape(d, h)).T
    gate = silu_gate(h1, h3)
    ffn = (gate.T @ np.asarray(w2, F32).reshape(d, h).T).T  # [d, seq]
    alpha = cfg.alpha()
    x_next = (np.asarray(x2_cf, F32).reshape(d, seq) + (ffn * alpha).astype(F32)).astype(F32)
    return {"x_next": x_next, "h1": h1.astype(F32), "h3": h3.astype(F32), "gate": gate}


def layer_forward(cfg: Config, lw: LayerW, x_cf: np.ndarray, seq: int, rope=None):
    """layer.rs:443-551 (forward): RMSNorm1 -> sdpaFwd -> woFwd -> x2 = x + alpha*o (vsma,
    layer.rs:784) -> RMSNorm2 -> ffnFused. Returns (x_next [dim*seq] channel-first, taps)."""
    d = cfg.dim
    xnorm, rms1 = rmsnorm_channel_first(x_cf, lw.gamma1, d, seq, cfg.norm_eps)
    s = sdpa_fwd(cfg, xnorm, lw.wq, lw.wk, lw.wv, seq, rope)
    o = dyn_matmul(s["attn"], lw.wo, cfg.q_dim, d, seq)
    x2 = vsma(o.reshape(-1), cfg.alpha(), np.asarray(x_cf, F32).reshape(-1))
    x2norm, rms2 = rmsnorm_channel_first(x2, lw.gamma2, d, seq, cfg.norm_eps)
    f = ffn_fused(cfg, x2norm, x2, lw.w1, lw.w3, lw.w2, seq)
    taps = dict(xnorm=xnorm, rms_inv1=rms1, o=o, x2=x2, x2norm=x2norm, rms_inv2=rms2, **s,
                h1=f["h1"], h3=f["h3"], gate=f["gate"])
    return f["x_next"].reshape(-1), taps


def softcap_forward(logits: np.ndarray, softcap: float) -> np.ndarray:
    """full_model.rs:234-239 / 388-393, in the reference's operation order:
    logits *= 1/c (vDSP sscal by the f32 reciprocal), t = tanh(logits),
    logits = t * c (vsmul). Dividing by c instead rounds differently whenever
    1/c is not a power of two."""
    c = F32(softcap)
    t = np.tanh((np.asarray(logits, F32) * (F32(1.0) / c)).astype(F32)).astype(F32)
    return (t * c).astype(F32)


def model_forward(cfg: Config, w: ModelW, tokens, targets=None, softcap: float = 0.0,
                  want_logits: bool = True, keep_taps=False):
    """full_model.rs:345-410 / 717-767 for one sequence: embedding + mtrans (201-202) ->
    layers (207-215) -> final RMSNorm (223) -> logits = XF^T E^T into zeroed buffer
    (228-230) -> softcap (234-239) -> CE (242-246). Returns dict(loss, losses, logits,
    x_final_cf, taps). keep_taps: False, True (every tap of every layer) or a
    collection of tap names to keep."""
    d, V = cfg.dim, cfg.vocab
    seq = len(tokens)
    x_row = embedding_forward(w.embed, d, tokens)
    x = mtrans(x_row, seq, d)  # [d, seq]
    rope = rope_table(seq, cfg.hd, cfg.rope_theta)
    taps = []
    for l in range(cfg.nlayers):
        x, t = layer_forward(cfg, w.layers[l], x, seq, rope)
        if keep_taps is True:
            taps.append(t)
        elif keep_taps:
            taps.append({k: t[k] for k in keep_taps})
    x_final, _ = rmsnorm_channel_first(x, w.gamma_final, d, seq, cfg.norm_eps)
    x_final_row = mtrans(x_final, d, seq)
    logits = sgemm_at(x_final_row, seq, d, w.embed, V, np.zeros(seq * V, F32))
    if softcap > 0.0:
        logits = softcap_forward(logits, softcap)
    out = {"logits": logits if want_logits else None, "x_final_cf": x_final, "taps": taps,
           "x_prenorm_cf": x}
    if targets is not None:
        total, losses = cross_entropy_batch(logits, targets, V)
        out["loss"] = F32(total / F32(seq))
        out["losses"] = losses
    return out


def forward_batch(cfg: Config, w: ModelW, tokens, targets=None, B: int = 1, softcap: float = 0.0,
                  want_logits: bool = True):
    """B > 1 is B independent B = 1 forwards (the reference has no batch dimension)."""
    tok = np.asarray(tokens).reshape(B, -1)
    tgt = None if targets is None else np.asarray(targets).reshape(B, -1)
    outs = [model_forward(cfg, w, tok[b], None if tgt is None else tgt[b], softcap, want_logits)
            for b in range(B)]
    res = {}
    if want_logits:
        res["logits"] = np.stack([o["logits"].reshape(tok.shape[1], cfg.vocab) for o in outs])
    if tgt is not None:
        res["losses"] = np.stack([o["losses"] for o in outs])
        res["loss"] = F32(res["losses"].astype(np.float64).mean())
    return res


class DecodeOracle:
    """Incremental single-sequence decode: steps 1-6 of the forward applied to one new column
    at position p, attending to the K'/V of positions <= p kept in a cache (the decode loop
    crates/metal-decode/src/lib.rs:3-4 plans; its result equals row p of model_forward over
    tokens[0..p])."""

    def __init__(self, cfg: Config, w: ModelW, ctx_max: int):
        self.cfg, self.w = cfg, w
        self.rope = rope_table(ctx_max, cfg.hd, cfg.rope_theta)
        L, KVH, hd = cfg.nlayers, cfg.kv_heads, cfg.hd
        self.k = np.zeros((L, KVH, ctx_max, hd), F32)
        self.v = np.zeros((L, KVH, ctx_max, hd), F32)
        self.pos = 0

    def prefill(self, tokens, targets=None) -> np.ndarray:
        """Full forward over the prompt (model_forward), keeping each layer's K'/V for
        positions [0, S); returns the last position's logits. The whole forward result
        (logits [S*vocab], and losses/loss when targets are given) stays in
        self.prefill_out."""
        cfg = self.cfg
        S = len(tokens)
        out = model_forward(cfg, self.w, tokens, targets, cfg.softcap, True,
                            keep_taps=("k_rope", "v"))
        for l, t in enumerate(out.pop("taps")):
            self.k[l, :, :S] = t["k_rope"].reshape(cfg.kv_heads, cfg.hd, S).transpose(0, 2, 1)
            self.v[l, :, :S] = t["v"].reshape(cfg.kv_heads, cfg.hd, S).transpose(0, 2, 1)
        self.pos = S
        self.prefill_out = out
        return out["logits"].reshape(S, cfg.vocab)[-1].copy()

    def step(self, token: int) -> np.ndarray:
        """Logits [vocab] for the token at position self.pos; appends its K'/V."""
        cfg, w, p = self.cfg, self.w, self.pos
        d, H, KVH, hd = cfg.dim, cfg.heads, cfg.kv_heads, cfg.hd
        x = embedding_forward(w.embed, d, [token]).reshape(d, 1)
        alpha = cfg.alpha()
        scale = F32(1.0) / np.sqrt(F32(hd))
        for l, lw in enumerate(w.layers):
            xn, _ = rmsnorm_channel_first(x, lw.gamma1, d, 1, cfg.norm_eps)
            xnt = xn.reshape(d, 1).T
            Qf = (xnt @ lw.wq.reshape(d, cfg.q_dim)).T
            Kf = (xnt @ lw.wk.reshape(d, cfg.kv_dim)).T
            Vf = (xnt @ lw.wv.reshape(d, cfg.kv_dim)).T
            Qr = rope_apply_cf(Qf, H, hd, 1, *self.rope, pos0=p).reshape(H, hd)
            Kr = rope_apply_cf(Kf, KVH, hd, 1, *self.rope, pos0=p).reshape(KVH, hd)
            self.k[l, :, p] = Kr
            self.v[l, :, p] = Vf.reshape(KVH, hd)
            rep = H // KVH
            K = self.k[l, :, :p + 1]  # [KVH, p+1, hd]
            Vc = self.v[l, :, :p + 1]
            if rep > 1:  # query head h reads kv head h // rep
                K = np.repeat(K, rep, axis=0)
                Vc = np.repeat(Vc, rep, axis=0)
            sc = np.matmul(K, Qr[:, :, None])[:, :, 0].astype(F32) * scale  # [H, p+1]
            pr = _softmax_last(sc)
            attn = np.matmul(pr[:, None, :], Vc)[:, 0, :].astype(F32).reshape(cfg.q_dim, 1)
            o = dyn_matmul(attn, lw.wo, cfg.q_dim, d, 1)
            x2 = vsma(o.reshape(-1), alpha, x.reshape(-1)).reshape(d, 1)
            x2n, _ = rmsnorm_channel_first(x2, lw.gamma2, d, 1, cfg.norm_eps)
            x = ffn_fused(cfg, x2n, x2, lw.w1, lw.w3, lw.w2, 1)["x_next"]
        xf, _ = rmsnorm_channel_first(x, w.gamma_final, d, 1, cfg.norm_eps)
        logits = sgemm_at(xf.reshape(1, d), 1, d, w.embed, cfg.vocab, np.zeros(cfg.vocab, F32))
        if cfg.softcap > 0:
            logits = softcap_forward(logits, cfg.softcap)
        self.pos += 1
        return logits.reshape(-1)
