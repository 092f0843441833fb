"""Pins for the CPU oracle (oracle/forward.py).

Each oracle function is checked against (a) the known-answer tests the
reference keeps next to the op (crates/engine/src/cpu/*.rs #[cfg(test)]
modules), (b) closed forms and invariants, and (c) an independent torch-CPU
fp32 implementation written with different primitives (complex-number RoPE,
F.scaled_dot_product_attention, F.cross_entropy). A plausible mistake — a
dropped term, a wrong RoPE sign or pair index, a transposed weight — fails at
least one of them (see test_planted_mistakes_are_caught).
"""
import math

import numpy as np
import pytest

import oracle as O

F32 = np.float32


def tiny_cfg(**kw):
    base = dict(dim=64, hidden=128, heads=4, kv_heads=4, hd=16, seq=12, nlayers=2, vocab=96,
                q_dim=64, kv_dim=64, gqa_ratio=1)
    base.update(kw)
    return O.Config(**base)


def tiny_weights(cfg, seed=0, std=0.05):
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


# ---- reference known answers (cpu/*.rs test modules) --------------------------

def test_embedding_forward_lookup():
    # cpu/embedding.rs:50-62
    table = np.array([1, 2, 3, 4, 5, 6], F32)
    out = O.embedding_forward(table, 2, [2, 0, 1])
    assert out.tolist() == [5.0, 6.0, 1.0, 2.0, 3.0, 4.0]


def test_embedding_roundtrip_identity():
    # cpu/embedding.rs:86-94
    table = np.array([10, 20, 30, 40], F32)
    assert O.embedding_forward(table, 2, [0, 1]).tolist() == table.tolist()


def test_rmsnorm_forward_unit_gamma():
    # cpu/rmsnorm.rs:244-256
    out, rms_inv = O.rmsnorm_forward(np.array([3.0, 4.0], F32), np.array([1.0, 1.0], F32))
    expected_rms = math.sqrt(12.5 + 1e-5)
    assert abs(rms_inv - 1 / expected_rms) < 1e-5
    assert abs(out[0] - 3 / expected_rms) < 1e-5
    assert abs(out[1] - 4 / expected_rms) < 1e-5


def test_rmsnorm_forward_with_gamma():
    # cpu/rmsnorm.rs:258-273
    x = np.array([1, 2, 3, 4], F32)
    out, rms_inv = O.rmsnorm_forward(x, np.full(4, 0.5, F32))
    e = 1 / math.sqrt(7.5 + 1e-5)
    assert abs(rms_inv - e) < 1e-5
    for i in range(4):
        assert abs(out[i] - x[i] * e * 0.5) < 1e-5


def test_rmsnorm_channel_first_matches_batch():
    # cpu/rmsnorm.rs:315-356: channel-first == per-token forward
    dim, seq = 4, 3
    gamma = np.array([1.5, 0.5, 2.0, 0.8], F32)
    x_cf = np.array([((i * 17 + 3) % 100) * 0.01 - 0.5 for i in range(dim * seq)], F32)
    out_cf, rms_cf = O.rmsnorm_channel_first(x_cf, gamma, dim, seq)
    xt = x_cf.reshape(dim, seq).T
    for s in range(seq):
        o, r = O.rmsnorm_forward(xt[s], gamma)
        assert abs(rms_cf[s] - r) < 1e-5
        np.testing.assert_allclose(out_cf.reshape(dim, seq)[:, s], o, atol=1e-5)


def test_rmsnorm_closed_form_constant_rows():
    # |x| constant c along a row => rms_inv = 1/sqrt(c^2 + eps); y = sign(x) * c * r * gamma
    dim, seq = 8, 5
    c = np.array([0.5, 1.0, 2.0, 3.0, 7.0], F32)
    signs = np.where(np.arange(dim) % 3 == 0, -1.0, 1.0).astype(F32)
    x = signs[:, None] * c[None, :]
    g = np.linspace(0.5, 2.0, dim).astype(F32)
    out, r = O.rmsnorm_channel_first(x.reshape(-1), g, dim, seq)
    np.testing.assert_allclose(r, 1 / np.sqrt(c.astype(np.float64) ** 2 + 1e-5), rtol=1e-6)
    np.testing.assert_allclose(out.reshape(dim, seq), signs[:, None] * c * r * g[:, None], rtol=1e-6)


def test_cross_entropy_known_answers():
    # cpu/cross_entropy.rs:102-118
    loss, _ = O.cross_entropy_forward(np.array([1, 2, 3, 4], F32), 3)
    assert 0.0 < loss < 2.0
    low, _ = O.cross_entropy_forward(np.array([1, 1, 1, 1], F32), 3)
    high, _ = O.cross_entropy_forward(np.array([0, 0, 0, 10], F32), 3)
    assert high < low


def test_cross_entropy_uniform_is_ln_vocab_and_brute_force():
    for V in (4, 97, 32000):
        loss, _ = O.cross_entropy_forward(np.zeros(V, F32), V // 2)
        assert abs(loss - math.log(V)) < 1e-5 * max(1, math.log(V))
    rng = np.random.default_rng(3)
    L = rng.normal(0, 3, size=(7, 50)).astype(F32)
    y = rng.integers(0, 50, size=7)
    total, losses = O.cross_entropy_batch(L, y, 50)
    for s in range(7):
        row = L[s].astype(np.float64)
        bf = math.log(sum(math.exp(v) for v in row)) - row[y[s]]
        assert abs(losses[s] - bf) < 1e-4
    assert abs(total - losses.astype(np.float64).sum()) < 1e-3


def test_silu_gate_known_answers():
    # cpu/silu.rs:52-69, 95-108
    assert abs(O.silu_gate(np.array([0.0], F32), np.array([1.0], F32))[0]) < 1e-6
    sig2 = 1 / (1 + math.exp(-2.0))
    assert abs(O.silu_gate(np.array([2.0], F32), np.array([1.0], F32))[0] - 2 * sig2) < 1e-6
    g = np.array([1.0, 2.0], F32)
    u = np.array([3.0, 4.0], F32)
    silu = g / (1 + np.exp(-g))
    np.testing.assert_allclose(O.silu_gate(g, u), silu * u, atol=1e-6)


def test_vsma_known_answer():
    # cpu/vdsp.rs:393-401
    assert O.vsma(np.array([1, 2, 3], F32), 2.0, np.array([10, 20, 30], F32)).tolist() == [12, 24, 36]


def test_sgemm_at_accumulates_and_brute_force():
    # cpu/vdsp.rs:287-302: C += A @ B^T with beta = 1
    rng = np.random.default_rng(1)
    a = rng.normal(size=(3, 5)).astype(F32)
    b = rng.normal(size=(4, 5)).astype(F32)
    c0 = np.ones((3, 4), F32)
    c = O.sgemm_at(a, 3, 5, b, 4, c0)
    for i in range(3):
        for j in range(4):
            assert abs(c[i, j] - (1 + sum(a[i, k] * b[j, k] for k in range(5)))) < 1e-5


def test_mtrans():
    a = np.arange(6, dtype=F32)
    assert O.mtrans(a, 2, 3).tolist() == [0, 3, 1, 4, 2, 5]


def test_dyn_matmul_one_hot_and_brute_force():
    ic, oc, seq = 6, 4, 3
    rng = np.random.default_rng(2)
    acts = rng.normal(size=(ic, seq)).astype(F32)
    w = np.zeros((ic, oc), F32)
    w[2, 1] = 1.0  # one-hot: out[1] = acts[2]
    out = O.dyn_matmul(acts, w, ic, oc, seq)
    np.testing.assert_array_equal(out[1], acts[2])
    assert not out[[0, 2, 3]].any()
    w = rng.normal(size=(ic, oc)).astype(F32)
    out = O.dyn_matmul(acts, w, ic, oc, seq)
    bf = [[sum(acts[i, s] * w[i, o] for i in range(ic)) for s in range(seq)] for o in range(oc)]
    np.testing.assert_allclose(out, bf, atol=1e-5)


# ---- RoPE ------------------------------------------------------------------------

def test_rope_identity_at_position_zero_and_norm_preserved():
    H, hd, seq = 3, 8, 10
    cos, sin = O.rope_table(seq, hd)
    x = np.random.default_rng(0).normal(size=(H * hd, seq)).astype(F32)
    y = O.rope_apply_cf(x, H, hd, seq, cos, sin)
    np.testing.assert_array_equal(y[:, 0], x[:, 0])
    xp = x.reshape(H, hd // 2, 2, seq)
    yp = y.reshape(H, hd // 2, 2, seq)
    np.testing.assert_allclose(np.hypot(yp[:, :, 0], yp[:, :, 1]), np.hypot(xp[:, :, 0], xp[:, :, 1]),
                               rtol=1e-5)


def test_rope_reference_inverse_undoes_forward():
    # layer.rs:1880-1897 (rope_backward_inplace) is the transpose of the rotation
    H, hd, seq = 2, 16, 33
    cos, sin = O.rope_table(seq, hd)
    x = np.random.default_rng(1).normal(size=(H * hd, seq)).astype(F32)
    y = O.rope_apply_cf(x, H, hd, seq, cos, sin)
    np.testing.assert_allclose(O.rope_backward_cf(y, H, hd, seq), x, atol=2e-5)


def test_rope_matches_complex_rotation_torch():
    torch = pytest.importorskip("torch")
    H, hd, seq = 2, 16, 20
    cos, sin = O.rope_table(seq, hd)
    x = np.random.default_rng(5).normal(size=(H * hd, seq)).astype(F32)
    y = O.rope_apply_cf(x, H, hd, seq, cos, sin)
    # Independent: pairs (2i, 2i+1) as complex numbers times e^{i p / base^(2i/hd)}.
    xt = torch.tensor(x.reshape(H, hd // 2, 2, seq)).permute(0, 3, 1, 2).contiguous()  # H,seq,hd/2,2
    z = torch.view_as_complex(xt.to(torch.float64))
    i = torch.arange(hd // 2, dtype=torch.float64)
    p = torch.arange(seq, dtype=torch.float64)
    ang = p[:, None] / (10000.0 ** (2 * i / hd))[None, :]
    yr = torch.view_as_real(z * torch.polar(torch.ones_like(ang), ang)[None])
    yref = yr.permute(0, 2, 3, 1).reshape(H * hd, seq).numpy()
    np.testing.assert_allclose(y, yref, atol=2e-4)


# ---- attention ---------------------------------------------------------------------

def _attn_only(cfg, seed=0, seq=None):
    seq = seq or cfg.seq
    rng = np.random.default_rng(seed)
    xn = rng.normal(size=(cfg.dim, seq)).astype(F32)
    wq = rng.normal(0, 0.2, size=(cfg.dim, cfg.q_dim)).astype(F32)
    wk = rng.normal(0, 0.2, size=(cfg.dim, cfg.kv_dim)).astype(F32)
    wv = rng.normal(0, 0.2, size=(cfg.dim, cfg.kv_dim)).astype(F32)
    return xn, wq, wk, wv, O.sdpa_fwd(cfg, xn, wq, wk, wv, seq)


def test_sdpa_matches_torch_sdpa():
    torch = pytest.importorskip("torch")
    import torch.nn.functional as Fn
    for cfg in (tiny_cfg(), tiny_cfg(kv_heads=2, kv_dim=32, gqa_ratio=2)):
        seq = cfg.seq
        xn, wq, wk, wv, out = _attn_only(cfg)
        q = torch.tensor(out["q_rope"]).reshape(cfg.heads, cfg.hd, seq).transpose(1, 2)
        k = torch.tensor(out["k_rope"]).reshape(cfg.kv_heads, cfg.hd, seq).transpose(1, 2)
        v = torch.tensor(out["v"]).reshape(cfg.kv_heads, cfg.hd, seq).transpose(1, 2)
        rep = cfg.heads // cfg.kv_heads
        k = k.repeat_interleave(rep, 0)
        v = v.repeat_interleave(rep, 0)
        a = Fn.scaled_dot_product_attention(q[None], k[None], v[None], is_causal=True)[0]
        ref = a.transpose(1, 2).reshape(cfg.q_dim, seq).numpy()
        np.testing.assert_allclose(out["attn"], ref, atol=2e-5)


def test_sdpa_single_position_returns_v_and_identical_keys_average():
    cfg = tiny_cfg(seq=1)
    _, _, _, _, out = _attn_only(cfg, seq=1)
    np.testing.assert_allclose(out["attn"], out["v"], atol=1e-6)
    # Wk = 0 => all scores 0 => causal mean of V[0..s]
    cfg = tiny_cfg()
    rng = np.random.default_rng(4)
    xn = rng.normal(size=(cfg.dim, cfg.seq)).astype(F32)
    wq = rng.normal(size=(cfg.dim, cfg.q_dim)).astype(F32)
    wv = rng.normal(size=(cfg.dim, cfg.kv_dim)).astype(F32)
    out = O.sdpa_fwd(cfg, xn, wq, np.zeros((cfg.dim, cfg.kv_dim), F32), wv, cfg.seq)
    v = out["v"]
    prefix_mean = np.cumsum(v, axis=1) / np.arange(1, cfg.seq + 1)[None, :]
    np.testing.assert_allclose(out["attn"], prefix_mean, atol=1e-5)


# ---- whole model -----------------------------------------------------------------

def _torch_forward(cfg, w, tokens, targets):
    """Independent fp32 forward: token-major torch ops, complex RoPE, torch SDPA,
    F.silu, F.cross_entropy."""
    import torch
    import torch.nn.functional as Fn
    T = torch.tensor
    S = len(tokens)
    E = T(w.embed).reshape(cfg.vocab, cfg.dim)
    x = E[torch.tensor(np.asarray(tokens, np.int64))]

    def rms(x, g):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + cfg.norm_eps) * T(g)

    i = torch.arange(cfg.hd // 2, dtype=torch.float64)
    ang = torch.arange(S, dtype=torch.float64)[:, None] / (cfg.rope_theta ** (2 * i / cfg.hd))[None]
    rot = torch.polar(torch.ones_like(ang), ang)

    def rope(t, nh):  # t [S, nh*hd]
        z = torch.view_as_complex(t.reshape(S, nh, cfg.hd // 2, 2).to(torch.float64).contiguous())
        return torch.view_as_real(z * rot[:, None]).reshape(S, nh * cfg.hd).float()

    alpha = float(cfg.alpha())
    for lw in w.layers:
        xn = rms(x, lw.gamma1)
        q = rope(xn @ T(lw.wq).reshape(cfg.dim, cfg.q_dim), cfg.heads)
        k = rope(xn @ T(lw.wk).reshape(cfg.dim, cfg.kv_dim), cfg.kv_heads)
        v = xn @ T(lw.wv).reshape(cfg.dim, cfg.kv_dim)
        qh = q.reshape(S, cfg.heads, cfg.hd).transpose(0, 1)
        rep = cfg.heads // cfg.kv_heads
        kh = k.reshape(S, cfg.kv_heads, cfg.hd).transpose(0, 1).repeat_interleave(rep, 0)
        vh = v.reshape(S, cfg.kv_heads, cfg.hd).transpose(0, 1).repeat_interleave(rep, 0)
        a = Fn.scaled_dot_product_attention(qh[None], kh[None], vh[None], is_causal=True)[0]
        a = a.transpose(0, 1).reshape(S, cfg.q_dim)
        x2 = x + alpha * (a @ T(lw.wo).reshape(cfg.q_dim, cfg.dim))
        x2n = rms(x2, lw.gamma2)
        g = Fn.silu(x2n @ T(lw.w1).reshape(cfg.dim, cfg.hidden)) * (x2n @ T(lw.w3).reshape(cfg.dim, cfg.hidden))
        x = x2 + alpha * (g @ T(lw.w2).reshape(cfg.dim, cfg.hidden).T)
    xf = rms(x, w.gamma_final)
    logits = xf @ E.T
    losses = Fn.cross_entropy(logits, torch.tensor(np.asarray(targets, np.int64)), reduction="none")
    return logits.numpy(), losses.numpy()


@pytest.mark.parametrize("gqa", [1, 2])
def test_model_forward_matches_independent_torch(gqa):
    pytest.importorskip("torch")
    cfg = tiny_cfg(kv_heads=4 // gqa, kv_dim=64 // gqa, gqa_ratio=gqa)
    w = tiny_weights(cfg)
    rng = np.random.default_rng(7)
    tok = rng.integers(0, cfg.vocab, cfg.seq + 1)
    out = O.model_forward(cfg, w, tok[:-1], tok[1:])
    logits, losses = _torch_forward(cfg, w, tok[:-1], tok[1:])
    np.testing.assert_allclose(out["logits"].reshape(cfg.seq, cfg.vocab), logits, atol=2e-5)
    np.testing.assert_allclose(out["losses"], losses, rtol=1e-5)
    assert abs(out["loss"] - losses.mean()) < 1e-5


def test_model_forward_init_loss_near_ln_vocab():
    # phase4_training.rs:84-100 (0 < loss < 20, ~ln V for small weights)
    cfg = tiny_cfg(vocab=512)
    w = tiny_weights(cfg, std=0.01)
    tok = np.arange(cfg.seq + 1) % cfg.vocab
    out = O.model_forward(cfg, w, tok[:-1], tok[1:])
    assert 0 < out["loss"] < 20
    assert abs(out["loss"] - math.log(cfg.vocab)) < 0.05


def test_softcap_bounds_logits():
    cfg = tiny_cfg()
    w = tiny_weights(cfg, std=0.5)
    tok = np.arange(cfg.seq + 1) % cfg.vocab
    raw = O.model_forward(cfg, w, tok[:-1], tok[1:])["logits"]
    capped = O.model_forward(cfg, w, tok[:-1], tok[1:], softcap=3.0)["logits"]
    assert np.abs(capped).max() < 3.0
    np.testing.assert_allclose(capped, 3.0 * np.tanh(raw / 3.0), atol=1e-5)


def test_softcap_uses_the_reference_operation_order():
    """full_model.rs:388-393 scales by the f32 reciprocal 1/c before tanh and
    multiplies by c after. For c = 3, x * fl(1/3) and x / 3 differ in fp32 for
    about a third of inputs; the forward oracle, the decode oracle and the
    backward oracle (which stores the same tanh for the softcap derivative)
    must all take the reciprocal route, bit for bit."""
    import oracle.backward as OB
    x = np.linspace(-40, 40, 4001, dtype=F32)
    recip = (x * (F32(1) / F32(3))).astype(F32)
    div = (x / F32(3)).astype(F32)
    assert (recip != div).mean() > 0.1  # the two orders are distinguishable here
    got = O.softcap_forward(x, 3.0)
    want = (np.tanh(recip).astype(F32) * F32(3)).astype(F32)
    np.testing.assert_array_equal(got, want)
    assert (got != (np.tanh(div).astype(F32) * F32(3)).astype(F32)).any()
    # whole-model paths: forward, decode and the backward's forward agree exactly
    cfg = tiny_cfg(softcap=3.0)
    w = tiny_weights(cfg, std=0.5)
    tok = np.arange(cfg.seq + 1) % cfg.vocab
    fwd = O.model_forward(cfg, w, tok[:-1], tok[1:], softcap=3.0)
    raw = O.model_forward(cfg, w, tok[:-1], tok[1:])["logits"]
    np.testing.assert_array_equal(fwd["logits"], O.softcap_forward(raw, 3.0))
    loss_b, _ = OB.model_forward_backward(cfg, w, tok[:-1], tok[1:], 3.0, 1.0)
    assert loss_b == pytest.approx(float(fwd["loss"]), rel=1e-6)


def test_decode_oracle_equals_prefill_rows():
    cfg = tiny_cfg()
    w = tiny_weights(cfg)
    tok = np.random.default_rng(9).integers(0, cfg.vocab, cfg.seq)
    full = O.model_forward(cfg, w, tok)["logits"].reshape(cfg.seq, cfg.vocab)
    dec = O.DecodeOracle(cfg, w, ctx_max=cfg.seq)
    for p in range(cfg.seq):
        np.testing.assert_allclose(dec.step(int(tok[p])), full[p], atol=2e-5)
    dec2 = O.DecodeOracle(cfg, w, ctx_max=cfg.seq)
    last = dec2.prefill(tok[:5])
    np.testing.assert_allclose(last, full[4], atol=2e-5)
    for p in range(5, cfg.seq):
        np.testing.assert_allclose(dec2.step(int(tok[p])), full[p], atol=2e-5)


def test_batch_is_independent_sequences():
    cfg = tiny_cfg()
    w = tiny_weights(cfg)
    tok = np.random.default_rng(11).integers(0, cfg.vocab, (3, cfg.seq + 1))
    res = O.forward_batch(cfg, w, tok[:, :-1], tok[:, 1:], B=3)
    for b in range(3):
        one = O.model_forward(cfg, w, tok[b, :-1], tok[b, 1:])
        np.testing.assert_array_equal(res["losses"][b], one["losses"])


def test_planted_mistakes_are_caught():
    """Plant plausible mistakes in a copy of the oracle's pieces and check the
    independent torch forward notices each one."""
    pytest.importorskip("torch")
    cfg = tiny_cfg()
    w = tiny_weights(cfg)
    tok = np.random.default_rng(13).integers(0, cfg.vocab, cfg.seq + 1)
    ref_logits, _ = _torch_forward(cfg, w, tok[:-1], tok[1:])
    good = O.model_forward(cfg, w, tok[:-1], tok[1:])["logits"].reshape(cfg.seq, cfg.vocab)
    assert np.abs(good - ref_logits).max() < 1e-4

    import oracle.forward as OF
    orig_rope, orig_mask, orig_silu = OF.rope_apply_cf, OF.causal_mask, OF.silu_gate

    def wrong_sign(x, h, hd, seq, cos, sin, pos0=0):
        return orig_rope(x, h, hd, seq, cos, -sin, pos0)

    def no_mask(seq):
        return np.zeros((seq, seq), F32)

    def silu_only(g, u):
        return (g / (1 + np.exp(-g)) + 0 * u).astype(F32)

    for name, fn in (("rope_apply_cf", wrong_sign), ("causal_mask", no_mask), ("silu_gate", silu_only)):
        setattr(OF, name, fn)
        try:
            bad = OF.model_forward(cfg, w, tok[:-1], tok[1:])["logits"].reshape(cfg.seq, cfg.vocab)
        finally:
            OF.rope_apply_cf, OF.causal_mask, OF.silu_gate = orig_rope, orig_mask, orig_silu
        assert np.abs(bad - ref_logits).max() > 1e-3, name
    # transposed W2 (a [dim, hidden] weight read as [hidden, dim]) on a square FFN
    cfg2 = tiny_cfg(hidden=64)
    w2 = tiny_weights(cfg2)
    ref2, _ = _torch_forward(cfg2, w2, tok[:-1], tok[1:])
    for lw in w2.layers:
        lw.w2 = np.ascontiguousarray(lw.w2.reshape(64, 64).T).reshape(-1)
    bad = O.model_forward(cfg2, w2, tok[:-1], tok[1:])["logits"].reshape(cfg2.seq, cfg2.vocab)
    assert np.abs(bad - ref2).max() > 1e-3
