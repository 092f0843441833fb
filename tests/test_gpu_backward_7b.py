"""The training backward at the full 7B shape (one sequence of 512 tokens),
checked through a size-independent property instead of the oracle: the
gradient's projection on a random direction u equals the central difference
of the loss along u,

    <dL/dgamma, u>  ~=  (L(gamma + eps u) - L(gamma - eps u)) / (2 eps).

The directions perturb fp32 parameters the device keeps unrounded -- the final
norm's gamma (gradient through the logits and the final RMSNorm) and layer 0's
attention-norm gamma (gradient through the backward of all 32 layers) -- so
the losses see exactly the perturbed values. (Layer 0's FFN-norm gamma is not
used: along random directions the loss is too curved in it for a wide eps
and too flat for a narrow one -- central differences moved 0.61 -> 0.72
between eps 0.04 and 0.005 against 0.714 analytic, with ~1.5% rounding noise
at the small end.) L is the device forward's mean loss
(hb_forward, per-position fp32 losses averaged in float64). The device
backward approximates the fp32 model's gradient and the device forward the
fp16-rounded model's loss, each to about 1e-3; eps per parameter is inside
the range where the central difference has converged (measured: layer 0's
gamma1 -2.29 analytic against -2.111 / -2.283 / -2.288 / -2.355 at eps 0.02 /
0.01 / 0.005 / 0.002 -- curvature above, fp16 rounding noise of the loss
below; the final gamma flat within 0.3% for eps 0.02..0.4). loss_scale is 1,
the hardest case for the fp16 dlogits (p/S ~ 6e-8 before their power-of-two
pre-scale).
"""
import numpy as np
import pytest

from rustane_amd import engine as E
from rustane_amd import hip_bridge as hb
from rustane_amd.engine import CompiledKernels, ModelConfig
from tests._util import tokens_for

pytestmark = pytest.mark.gpu

REL_TOL = 2e-2
EPS = {"gamma_final": 0.05, "gamma1": 0.01}


@pytest.fixture(scope="module")
def trained_7b(gpu):
    cfg = ModelConfig.llama_7b(seq=512)
    k = CompiledKernels.compile(cfg)
    k.init_synthetic(1234, 0.02)
    opt = hb.Optimizer(k.model, E.TrainConfig())
    tok = tokens_for(cfg, 513, seed=77)
    opt.zero_grads()
    loss = opt.forward_backward(tok[:-1], tok[1:], 1, 512, 1.0)
    print(f"7B training forward+backward: mean loss {loss:.5f}", flush=True)
    yield cfg, k, opt, tok
    opt.close()
    k.model.close()


def _loss(cfg, k, tok):
    losses = E.forward_losses(cfg, k, None, tok[:-1], tok[1:])
    return float(np.mean(np.asarray(losses, np.float64)))


def _check(name, g, u, lp, lm, eps):
    fd = (lp - lm) / (2 * eps)
    an = float(np.dot(np.asarray(g, np.float64), np.asarray(u, np.float64)))
    print(f"{name}: <g,u> {an:.6e}  central difference {fd:.6e}  rel {abs(an - fd) / abs(fd):.2e}", flush=True)
    assert abs(an - fd) <= REL_TOL * abs(fd), (name, an, fd)


def test_final_gamma_directional_derivative(trained_7b):
    cfg, k, opt, tok = trained_7b
    _, g = opt.download_embed(hb.Optimizer.GRADS)
    embed, gf = opt.download_embed(hb.Optimizer.WEIGHTS)
    u = np.random.default_rng(5).standard_normal(cfg.dim).astype(np.float32)
    eps = EPS["gamma_final"]
    try:
        k.model.upload_embed(embed, gf + np.float32(eps) * u)
        lp = _loss(cfg, k, tok)
        k.model.upload_embed(embed, gf - np.float32(eps) * u)
        lm = _loss(cfg, k, tok)
    finally:
        k.model.upload_embed(embed, gf)
    _check("gamma_final", g, u, lp, lm, eps)


def test_layer0_gamma1_directional_derivative(trained_7b):
    cfg, k, opt, tok = trained_7b
    which = "gamma1"
    g = opt.download_layer(0, hb.Optimizer.GRADS)[which]
    w = opt.download_layer(0, hb.Optimizer.WEIGHTS)
    u = np.random.default_rng(6).standard_normal(cfg.dim).astype(np.float32)
    base = w[which].copy()

    def upload(gamma):
        lw = E.LayerWeights(**{**w, which: gamma})
        k.model.upload_layer(0, lw)

    eps = EPS[which]
    try:
        upload(base + np.float32(eps) * u)
        lp = _loss(cfg, k, tok)
        upload(base - np.float32(eps) * u)
        lm = _loss(cfg, k, tok)
    finally:
        upload(base)
    _check(f"layer 0 {which}", g, u, lp, lm, eps)


def test_gradient_norm_from_tile_sums_matches_full_pass(trained_7b):
    """The norm hb_opt_grad_norm assembles from the backward's per-tile sums of
    squares (fp32 per weight-gradient tile, thousands of slots at 7B) against
    the full fp64 pass over the arena, which it takes once the raw arena
    pointer has been handed out."""
    cfg, k, opt, tok = trained_7b
    from_tiles = opt.grad_norm()
    opt.grad_arena()  # the next norm reads the whole arena
    full = opt.grad_norm()
    print(f"7B gradient norm: per-tile sums {from_tiles:.9e}, full pass {full:.9e}", flush=True)
    assert np.isfinite(full) and full > 0
    assert abs(from_tiles - full) <= 1e-5 * full, (from_tiles, full)
