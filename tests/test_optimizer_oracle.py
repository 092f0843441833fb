"""Pins for the optimizer oracle (oracle/optimizer.py).

(a) The reference's own AdamW tests (crates/engine/src/cpu/adam.rs:134-182),
(b) closed forms (the first bias-corrected step is lr * (sign(g) + wd p), the
schedule's warmup/cosine end points, a 3-4-5 gradient norm), (c) a float64
brute force of the same formula, (d) the reference's two formulations of the
step (multi-pass cpu/adam.rs:37-85 and fused 95-132) agreeing, and (e) planted
mistakes -- a dropped bias correction, weight decay on the gammas, the learning
rate groups swapped -- each caught by one of them.
"""
import math

import numpy as np
import pytest

import oracle.optimizer as OP

F32 = np.float32


def _adam_default():
    """AdamConfig::default (cpu/adam.rs:20-28)."""
    return dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01)


# ---- (a) cpu/adam.rs test module ------------------------------------------------

def test_step_moves_toward_minimum():
    c = _adam_default()
    p, g = np.full(4, 5.0, F32), np.ones(4, F32)
    m, v = np.zeros(4, F32), np.zeros(4, F32)
    before = p.sum()
    for t in range(1, 11):
        OP.step(p, g, m, v, t, c["lr"], c["beta1"], c["beta2"], c["eps"], c["weight_decay"])
    assert p.sum() < before


def test_zero_grad_only_weight_decay():
    c = dict(_adam_default(), weight_decay=0.1)
    p, g = np.ones(2, F32), np.zeros(2, F32)
    m, v = np.zeros(2, F32), np.zeros(2, F32)
    OP.step(p, g, m, v, 1, c["lr"], c["beta1"], c["beta2"], c["eps"], c["weight_decay"])
    assert p[0] < 1.0
    np.testing.assert_allclose(p, 1.0 - 1e-3 * 0.1, rtol=1e-6)


def test_momentum_accumulates():
    c = dict(_adam_default(), weight_decay=0.0)
    p, g = np.zeros(2, F32), np.ones(2, F32)
    m, v = np.zeros(2, F32), np.zeros(2, F32)
    OP.step(p, g, m, v, 1, c["lr"], c["beta1"], c["beta2"], c["eps"], c["weight_decay"])
    assert abs(m[0] - 0.1) < 1e-6 and abs(v[0] - 0.001) < 1e-6


# ---- (b), (c), (d) --------------------------------------------------------------

def _f64_step(p, g, m, v, t, lr, b1, b2, eps, wd, gs):
    g = g.astype(np.float64) * gs
    m = b1 * m.astype(np.float64) + (1 - b1) * g
    v = b2 * v.astype(np.float64) + (1 - b2) * g * g
    upd = (m / (1 - b1 ** t)) / (np.sqrt(v / (1 - b2 ** t)) + eps)
    return p.astype(np.float64) - lr * (upd + wd * p.astype(np.float64)), m, v


def test_fused_step_matches_float64_and_multipass_form():
    rng = np.random.default_rng(1)
    n = 4096
    p = rng.standard_normal(n).astype(F32)
    m = (rng.standard_normal(n) * 1e-3).astype(F32)
    v = (rng.random(n) * 1e-5).astype(F32)
    g = (rng.standard_normal(n) * 1e-2).astype(F32)
    for t in (1, 2, 7, 100):
        pf, mf, vf = p.copy(), m.copy(), v.copy()
        OP.step_fused(pf, g, mf, vf, t, 3e-4, 0.9, 0.95, 1e-8, 0.1, 1.0)
        p64, m64, v64 = _f64_step(p, g, m, v, t, 3e-4, 0.9, 0.95, 1e-8, 0.1, 1.0)
        np.testing.assert_allclose(pf, p64, rtol=2e-7, atol=1e-9)
        # b1*m + (1-b1)*g cancels where the two have opposite signs: bound the
        # error by the operands' size (a few fp32 ulps of |m| + |g|), not by |m_new|
        np.testing.assert_allclose(mf, m64, rtol=1e-6, atol=4e-7 * 1e-2)
        np.testing.assert_allclose(vf, v64, rtol=1e-6, atol=4e-7 * 1e-5)
        pm, mm, vm = p.copy(), m.copy(), v.copy()
        OP.step(pm, g, mm, vm, t, 3e-4, 0.9, 0.95, 1e-8, 0.1)
        np.testing.assert_array_equal(mm, mf)  # same two products and one sum
        np.testing.assert_allclose(vm, vf, rtol=3e-7)  # (1-b2)*g*g associates differently
        np.testing.assert_allclose(pm, pf, rtol=1e-6, atol=1e-10)


def test_grad_scale_is_applied_to_the_gradient():
    rng = np.random.default_rng(2)
    p, g = rng.standard_normal(64).astype(F32), rng.standard_normal(64).astype(F32)
    a = [p.copy(), np.zeros(64, F32), np.zeros(64, F32)]
    b = [p.copy(), np.zeros(64, F32), np.zeros(64, F32)]
    OP.step_fused(a[0], g, a[1], a[2], 3, 1e-3, 0.9, 0.95, 1e-8, 0.1, 0.25)
    OP.step_fused(b[0], (g * F32(0.25)).astype(F32), b[1], b[2], 3, 1e-3, 0.9, 0.95, 1e-8, 0.1, 1.0)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_first_step_closed_form():
    """t = 1 from zero moments: m_hat = g, v_hat = g^2, so p -= lr (g/(|g|+eps) + wd p)."""
    rng = np.random.default_rng(3)
    p = rng.standard_normal(256).astype(F32)
    g = (rng.standard_normal(256) * 1e-2).astype(F32)
    q, m, v = p.copy(), np.zeros(256, F32), np.zeros(256, F32)
    OP.step_fused(q, g, m, v, 1, 1e-3, 0.9, 0.95, 1e-8, 0.1, 1.0)
    expect = p - 1e-3 * (g / (np.abs(g) + 1e-8) + 0.1 * p)
    np.testing.assert_allclose(q, expect, rtol=1e-6, atol=1e-9)


def test_powi_matches_exact_powers():
    for b in (0.9, 0.95, 0.999):
        assert OP.powi_f32(b, 0) == 1.0
        assert OP.powi_f32(b, 1) == F32(b)
        assert OP.powi_f32(b, 2) == F32(F32(b) * F32(b))
        for t in (3, 10, 100):
            # each squaring doubles the relative error so far: about t * 2^-24 in all
            exact = float(F32(b)) ** t
            assert abs(float(OP.powi_f32(b, t)) - exact) <= t * 2.0 ** -23 * exact


def test_learning_rate_end_points():
    tc = OP.TrainConfig()
    assert OP.learning_rate(0, tc) == F32(F32(3e-4) / F32(100))
    assert OP.learning_rate(99, tc) == F32(3e-4)
    assert abs(OP.learning_rate(100, tc) - 3e-4) <= 1e-10           # cos(0) = 1
    assert abs(OP.learning_rate(10000, tc) - 3e-5) <= 1e-10         # cos(pi) = -1
    mid = 100 + (10000 - 100) // 2
    assert abs(OP.learning_rate(mid, tc) - (3e-4 + 3e-5) / 2) <= 1e-9
    lrs = [OP.learning_rate(s, tc) for s in range(100, 10001, 99)]
    assert all(a >= b for a, b in zip(lrs, lrs[1:]))                 # monotone decay


def _tiny_state(rng, layers=2, d=8, h=16, V=12):
    def t(*s):
        return rng.standard_normal(int(np.prod(s))).astype(F32)
    shapes = dict(wq=d * d, wk=d * d, wv=d * d, wo=d * d, w1=d * h, w3=d * h, w2=d * h, gamma1=d, gamma2=d)
    return {"embed": t(V, d), "gamma_final": t(d),
            "layers": [{k: t(n) for k, n in shapes.items()} for _ in range(layers)]}


def test_grad_norm_and_clip_known_answer():
    rng = np.random.default_rng(4)
    g = OP.zeros_like_state(_tiny_state(rng))
    g["embed"][3] = 3.0
    g["layers"][1]["w2"][5] = 4.0
    assert OP.grad_norm(g) == 5.0
    assert OP.clip_grads(g, 1.0) == 5.0
    assert abs(OP.grad_norm(g) - 1.0) < 1e-7
    assert abs(g["embed"][3] - 0.6) < 1e-7 and abs(g["layers"][1]["w2"][5] - 0.8) < 1e-7
    assert OP.clip_grads(g, 10.0) < 10.0 and abs(g["embed"][3] - 0.6) < 1e-7  # below max: unchanged


def test_combined_scale_descale_or_clip():
    tc = OP.TrainConfig(accum_steps=10, loss_scale=256.0, grad_clip=1.0)
    gsc = F32(1.0) / F32(2560.0)
    assert OP.combined_scale(100.0, tc) == gsc                       # 100/2560 < 1
    assert OP.combined_scale(5120.0, tc) == F32(F32(1.0) / F32(5120.0))  # 2 > 1: clip


def test_update_weights_groups():
    """Zero gradients: only weight decay moves anything, and only the matrices
    have it; with a gradient, each group moves at its own learning rate."""
    rng = np.random.default_rng(5)
    w = _tiny_state(rng)
    w0 = {"embed": w["embed"].copy(), "gamma_final": w["gamma_final"].copy(),
          "layers": [{k: a.copy() for k, a in lw.items()} for lw in w["layers"]]}
    tc = OP.TrainConfig()
    g = OP.zeros_like_state(w)
    opt = {"m": OP.zeros_like_state(w), "v": OP.zeros_like_state(w)}
    OP.update_weights(w, g, opt, 1, 1e-3, tc, 1.0)
    np.testing.assert_array_equal(w["embed"], w0["embed"])
    np.testing.assert_array_equal(w["gamma_final"], w0["gamma_final"])
    for lw, l0 in zip(w["layers"], w0["layers"]):
        np.testing.assert_array_equal(lw["gamma1"], l0["gamma1"])
        np.testing.assert_allclose(lw["wq"], l0["wq"] * (1 - 1e-3 * 0.05 * 0.1), rtol=1e-6)
    # unit gradients on a zero state: first-step moves of lr*scale per group
    w = OP.zeros_like_state(w)
    g = _tiny_state(rng)
    for d in [g] + g["layers"]:
        for k in d:
            if isinstance(d[k], np.ndarray):
                d[k][:] = 1.0
    opt = {"m": OP.zeros_like_state(w), "v": OP.zeros_like_state(w)}
    OP.update_weights(w, g, opt, 1, 1e-3, tc, 1.0)
    np.testing.assert_allclose(w["embed"], -1e-3 * 5.0, rtol=1e-5)
    np.testing.assert_allclose(w["gamma_final"], -1e-3, rtol=1e-5)
    np.testing.assert_allclose(w["layers"][0]["w1"], -1e-3 * 0.05, rtol=1e-5)
    np.testing.assert_allclose(w["layers"][1]["gamma2"], -1e-3, rtol=1e-5)


def test_planted_mistakes_are_caught():
    rng = np.random.default_rng(6)
    p = rng.standard_normal(256).astype(F32)
    g = (rng.standard_normal(256) * 1e-2).astype(F32)
    orig = OP.bias_corrections

    def no_bias_correction(b1, b2, t):
        return F32(1.0), F32(1.0)

    OP.bias_corrections = no_bias_correction
    try:
        with pytest.raises(AssertionError):
            test_first_step_closed_form()
    finally:
        OP.bias_corrections = orig
    # weight decay applied to gammas, or the embed/matrix learning rates swapped
    orig_update = OP.update_weights

    def decay_everything(weights, grads, opt, t, lr, tc, gs):
        tc2 = OP.TrainConfig(**{**tc.__dict__, "matrix_lr_scale": tc.embed_lr_scale,
                                "embed_lr_scale": tc.matrix_lr_scale})
        return orig_update(weights, grads, opt, t, lr, tc2, gs)

    OP.update_weights = decay_everything
    try:
        with pytest.raises(AssertionError):
            test_update_weights_groups()
    finally:
        OP.update_weights = orig_update
    # the (1 - beta2) * g * g term dropped to (1 - beta2) * g
    q, m, v = p.copy(), np.zeros(256, F32), np.zeros(256, F32)
    OP.step_fused(q, g, m, v, 2, 1e-3, 0.9, 0.95, 1e-8, 0.1, 1.0)
    p64, _, _ = _f64_step(p, g, np.zeros(256), np.zeros(256), 2, 1e-3, 0.9, 0.95, 1e-8, 0.1, 1.0)
    v_bad = (1 - 0.95) * g.astype(np.float64)
    upd_bad = (0.1 * g / (1 - 0.81)) / (np.sqrt(np.abs(v_bad) / (1 - 0.9025)) + 1e-8)
    assert np.abs((p - 1e-3 * (upd_bad + 0.1 * p)) - q).max() > 1e-5
    np.testing.assert_allclose(q, p64, rtol=2e-7, atol=1e-9)
