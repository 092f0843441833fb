"""Pins for the backward oracle (oracle/backward.py).

(a) The reference's own gradient tests: cpu/rmsnorm.rs:276-310 (RMSNorm dx
against a numerical gradient on its input values) and cpu/cross_entropy.rs:
120-155 (softmax - onehot sums to zero, matches a numerical gradient);
(b) every weight gradient of the whole model against torch autograd in
float64 on an independent restatement of the forward (token-major torch ops,
complex-number RoPE), for MHA, GQA and softcap; (c) planted mistakes -- the
softmax-backward row sum dropped, the RoPE inverse's sign flipped, the
residual alpha left out of the FFN branch -- each caught by (b).
"""
import numpy as np
import pytest

import oracle as O
import oracle.backward as OB

F32 = np.float32


def test_rmsnorm_backward_numerical_gradient():
    """cpu/rmsnorm.rs:276-310 on the same values (dim 4, one position, dy = 1)."""
    x = np.array([1.0, -2.0, 3.0, -0.5], F32)
    gamma = np.array([1.0, 0.5, 2.0, 1.5], F32)
    _, r = O.rmsnorm_channel_first(x, gamma, 4, 1)
    dx, dg = OB.rmsnorm_backward_cf(np.ones(4, F32), x, gamma, r, 4, 1)
    f = lambda v: O.rmsnorm_channel_first(v, gamma, 4, 1)[0].astype(np.float64).sum()
    for i in range(4):
        e = np.zeros(4, F32)
        e[i] = 1e-3
        num = (f(x + e) - f(x - e)) / 2e-3
        assert abs(dx[i] - num) < 1e-2
    # dgamma = dy * x_hat
    np.testing.assert_allclose(dg, x * r[0], rtol=1e-6)


def test_cross_entropy_backward_sums_to_zero_and_matches_numerical():
    """cpu/cross_entropy.rs:120-155 (one position, no 1/seq scale)."""
    logits = np.array([2.0, -1.0, 0.5, 1.5], F32)
    total, d = OB.cross_entropy_fwd_bwd(logits, [2], 4, F32(1.0))
    assert abs(d.sum()) < 1e-6
    for i in range(4):
        p, m = logits.copy(), logits.copy()
        p[i] += 1e-3
        m[i] -= 1e-3
        num = (O.cross_entropy_forward(p, 2)[0] - O.cross_entropy_forward(m, 2)[0]) / 2e-3
        assert abs(d[i] - num) < 5e-3


def _cfg(**kw):
    base = dict(dim=64, hidden=96, heads=4, kv_heads=4, hd=16, seq=12, nlayers=2, vocab=80,
                q_dim=64, kv_dim=64, gqa_ratio=1)
    base.update(kw)
    return O.Config(**base)


def _weights(cfg, seed=0, std=0.08):
    rng = np.random.default_rng(seed)
    n = lambda *s: rng.normal(0, std, size=int(np.prod(s))).astype(F32)
    layers = [O.LayerW(wq=n(cfg.dim, cfg.q_dim), wk=n(cfg.dim, cfg.kv_dim), wv=n(cfg.dim, cfg.kv_dim),
                       wo=n(cfg.q_dim, cfg.dim), w1=n(cfg.dim, cfg.hidden), w3=n(cfg.dim, cfg.hidden),
                       w2=n(cfg.dim, cfg.hidden),
                       gamma1=(1 + 0.1 * rng.standard_normal(cfg.dim)).astype(F32),
                       gamma2=(1 + 0.1 * rng.standard_normal(cfg.dim)).astype(F32))
              for _ in range(cfg.nlayers)]
    return O.ModelW(embed=n(cfg.vocab, cfg.dim), layers=layers,
                    gamma_final=(1 + 0.1 * rng.standard_normal(cfg.dim)).astype(F32))


def _torch_grads(cfg, w, tokens, targets, softcap, loss_scale):
    """Independent float64 forward in torch; gradients of loss_scale * mean CE."""
    import torch
    import torch.nn.functional as Fn
    D = torch.float64
    S = len(tokens)
    P = {}

    def par(name, a, shape):
        t = torch.tensor(np.asarray(a, np.float64).reshape(shape), dtype=D, requires_grad=True)
        P[name] = t
        return t

    E = par("embed", w.embed, (cfg.vocab, cfg.dim))
    gf = par("gamma_final", w.gamma_final, (cfg.dim,))
    x = E[torch.tensor(np.asarray(tokens, np.int64))]
    i = torch.arange(cfg.hd // 2, dtype=D)
    ang = torch.arange(S, dtype=D)[:, None] / (cfg.rope_theta ** (2 * i / cfg.hd))[None]
    rot = torch.polar(torch.ones_like(ang), ang)

    def rms(x, g):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.norm_eps) * g

    def rope(t, nh):
        z = torch.view_as_complex(t.reshape(S, nh, cfg.hd // 2, 2).contiguous())
        return torch.view_as_real(z * rot[:, None]).reshape(S, nh * cfg.hd)

    alpha = float(cfg.alpha())
    mask = torch.triu(torch.full((S, S), float("-inf"), dtype=D), 1)
    for l, lw in enumerate(w.layers):
        L = {k: par(f"{l}.{k}", getattr(lw, k), s) for k, s in
             (("wq", (cfg.dim, cfg.q_dim)), ("wk", (cfg.dim, cfg.kv_dim)), ("wv", (cfg.dim, cfg.kv_dim)),
              ("wo", (cfg.q_dim, cfg.dim)), ("w1", (cfg.dim, cfg.hidden)), ("w3", (cfg.dim, cfg.hidden)),
              ("w2", (cfg.dim, cfg.hidden)), ("gamma1", (cfg.dim,)), ("gamma2", (cfg.dim,)))}
        xn = rms(x, L["gamma1"])
        q = rope(xn @ L["wq"], cfg.heads).reshape(S, cfg.heads, cfg.hd).transpose(0, 1)
        k = rope(xn @ L["wk"], cfg.kv_heads).reshape(S, cfg.kv_heads, cfg.hd).transpose(0, 1)
        v = (xn @ L["wv"]).reshape(S, cfg.kv_heads, cfg.hd).transpose(0, 1)
        rep = cfg.heads // cfg.kv_heads
        k, v = k.repeat_interleave(rep, 0), v.repeat_interleave(rep, 0)
        p = torch.softmax(q @ k.transpose(1, 2) / np.sqrt(cfg.hd) + mask, dim=-1)
        a = (p @ v).transpose(0, 1).reshape(S, cfg.q_dim)
        x2 = x + alpha * (a @ L["wo"])
        x2n = rms(x2, L["gamma2"])
        x = x2 + alpha * ((Fn.silu(x2n @ L["w1"]) * (x2n @ L["w3"])) @ L["w2"].T)
    logits = rms(x, gf) @ E.T
    if softcap > 0:
        logits = softcap * torch.tanh(logits / softcap)
    loss = Fn.cross_entropy(logits, torch.tensor(np.asarray(targets, np.int64)))
    (loss * loss_scale).backward()
    g = {k: t.grad.numpy().reshape(-1) for k, t in P.items()}
    return float(loss.detach()), g


def _check(cfg, w, softcap=0.0, loss_scale=256.0, seed=1):
    pytest.importorskip("torch")
    rng = np.random.default_rng(seed)
    tok = rng.integers(0, cfg.vocab, cfg.seq + 1)
    tok[5] = tok[2]  # a repeated input token: its embedding rows add up
    loss, grads = OB.model_forward_backward(cfg, w, tok[:-1], tok[1:], softcap, loss_scale)
    tl, tg = _torch_grads(cfg, w, tok[:-1], tok[1:], softcap, loss_scale)
    assert abs(loss - tl) < 1e-5 * tl
    pairs = [("embed", grads["embed"]), ("gamma_final", grads["gamma_final"])]
    for l, lg in enumerate(grads["layers"]):
        pairs += [(f"{l}.{k}", lg[k]) for k in OB.LAYER_TENSORS]
    worst = 0.0
    for name, ours in pairs:
        ref = tg[name]
        err = np.abs(ours - ref).max() / np.abs(ref).max()
        worst = max(worst, err)
        assert err < 2e-4, (name, err)
    return worst


def test_model_gradients_match_torch_autograd_mha():
    cfg = _cfg()
    _check(cfg, _weights(cfg))


def test_model_gradients_match_torch_autograd_gqa():
    cfg = _cfg(heads=4, kv_heads=2, kv_dim=32, gqa_ratio=2)
    _check(cfg, _weights(cfg, seed=2))


def test_model_gradients_match_torch_autograd_softcap():
    cfg = _cfg()
    _check(cfg, _weights(cfg, seed=3, std=0.3), softcap=0.5)


def test_planted_mistakes_are_caught():
    pytest.importorskip("torch")
    cfg = _cfg()
    w = _weights(cfg, seed=4)
    orig_sdpa, orig_rope = OB.sdpa_backward, OB.rope_backward_cf

    def no_row_sum(cfg_, q, k, v, da, seq):
        """ds = probs * dp * scale: the '- sum(probs * dp)' term of sdpa_bwd.rs:140-146 dropped."""
        H, hd = cfg_.heads, cfg_.hd
        scale = F32(1.0) / np.sqrt(F32(hd))
        qh = q.reshape(H, hd, seq).transpose(0, 2, 1)
        kh = k.reshape(H, hd, seq).transpose(0, 2, 1)
        vh = v.reshape(H, hd, seq).transpose(0, 2, 1)
        dh = da.reshape(H, hd, seq).transpose(0, 2, 1)
        sc = (qh @ kh.transpose(0, 2, 1)) * scale + O.causal_mask(seq)[None]
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        ds = p * (dh @ vh.transpose(0, 2, 1)) * scale
        cf = lambda t: np.ascontiguousarray(t.transpose(0, 2, 1)).reshape(H * hd, seq).astype(F32)
        return cf(ds @ kh), cf(ds.transpose(0, 2, 1) @ qh), cf(p.transpose(0, 2, 1) @ dh)

    def forward_rotation(dx, heads, hd, seq, theta=10000.0):
        """The forward RoPE applied to the gradient instead of its inverse."""
        return O.rope_apply_cf(dx, heads, hd, seq, *O.rope_table(seq, hd, theta))

    for name, fn in (("sdpa_backward", no_row_sum), ("rope_backward_cf", forward_rotation)):
        setattr(OB, name, fn)
        try:
            with pytest.raises(AssertionError):
                _check(cfg, w)
        finally:
            OB.sdpa_backward, OB.rope_backward_cf = orig_sdpa, orig_rope
    # alpha missing on the FFN branch: scale dffn by 1 instead of alpha
    orig_layer = OB.layer_backward

    def no_alpha(cfg_, lw, taps, x_in, dy, seq):
        c2 = O.Config(**{**cfg_.__dict__, "residual_alpha": 1.0})
        return orig_layer(c2, lw, taps, x_in, dy, seq)

    OB.layer_backward = no_alpha
    try:
        with pytest.raises(AssertionError):
            _check(cfg, w)
    finally:
        OB.layer_backward = orig_layer
