"""Optimizer on the GPU through the C ABI (hb_opt_*), against the oracle
(oracle/optimizer.py) on identical fp32 weights and gradients.

The fused AdamW kernel evaluates the reference's expression (cpu/adam.rs:119-131)
in the same order with every operation rounded to fp32, so weights and both
moments must match the oracle bit for bit; the gradient norm (an fp64 sum on
both sides, in different orders) and everything derived from it must agree to
fp32 rounding.
"""
import numpy as np
import pytest

import oracle as O
import oracle.optimizer as OP
from rustane_amd import engine as E
from rustane_amd import hip_bridge as hb
from rustane_amd.engine import CompiledKernels, ModelConfig, ModelWeights
from tests._util import F32, f16_round, oracle_cfg, tiny_config, tokens_for

pytestmark = pytest.mark.gpu


def _state_of(w: ModelWeights):
    return {"embed": np.array(w.embed, F32), "gamma_final": np.array(w.gamma_final, F32),
            "layers": [{k: np.array(getattr(lw, k), F32) for k in OP.LAYER_TENSORS} for lw in w.layers]}


def _random_grads(like, seed, std):
    rng = np.random.default_rng(seed)
    def r(a):
        return (rng.standard_normal(a.size) * std).astype(F32)
    return {"embed": r(like["embed"]), "gamma_final": r(like["gamma_final"]),
            "layers": [{k: r(a) for k, a in lw.items()} for lw in like["layers"]]}


def _upload_grads(opt, g):
    for l, lg in enumerate(g["layers"]):
        opt.upload_grads_layer(l, lg)
    opt.upload_grads_embed(g["embed"], g["gamma_final"])


def _device_state(opt, which, nlayers):
    e, gf = opt.download_embed(which)
    return {"embed": e, "gamma_final": gf,
            "layers": [opt.download_layer(l, which) for l in range(nlayers)]}


def _assert_state_equal(dev, ref, what):
    np.testing.assert_array_equal(dev["embed"], ref["embed"], err_msg=f"{what} embed")
    np.testing.assert_array_equal(dev["gamma_final"], ref["gamma_final"], err_msg=f"{what} gamma_final")
    for l, (a, b) in enumerate(zip(dev["layers"], ref["layers"])):
        for k in OP.LAYER_TENSORS:
            np.testing.assert_array_equal(a[k], b[k], err_msg=f"{what} layer {l} {k}")


@pytest.fixture
def tiny_opt(gpu):
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=3, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    yield cfg, k, w, st
    st.close()


def test_update_weights_bit_exact_three_steps(tiny_opt):
    cfg, k, w, st = tiny_opt
    tc = OP.TrainConfig()
    ref = _state_of(w)
    mom = {"m": OP.zeros_like_state(ref), "v": OP.zeros_like_state(ref)}
    _assert_state_equal(_device_state(st.opt, 0, cfg.nlayers), ref, "uploaded master")
    for t in (1, 2, 3):
        g = _random_grads(ref, seed=10 + t, std=1e-2)
        _upload_grads(st.opt, g)
        lr = OP.learning_rate(t + 40, tc)
        OP.update_weights(ref, g, mom, t, lr, tc, 0.37)
        st.opt.update_weights(t, float(lr), 0.37)
        print(f"t={t}: lr={lr:.6e}", flush=True)
    _assert_state_equal(_device_state(st.opt, 0, cfg.nlayers), ref, "weights")
    _assert_state_equal(_device_state(st.opt, 1, cfg.nlayers), mom["m"], "m")
    _assert_state_equal(_device_state(st.opt, 2, cfg.nlayers), mom["v"], "v")


@pytest.mark.parametrize("std,clipped", [(1e-2, False), (100.0, True)])
def test_optimizer_step_norm_and_clip_decision(tiny_opt, std, clipped):
    """train_step's tail (full_model.rs:697-711) with the clip decided on the
    device: small gradients are descaled by 1/(accum*loss_scale), large ones
    clipped to grad_clip."""
    cfg, k, w, st = tiny_opt
    tc = OP.TrainConfig()
    ref = _state_of(w)
    mom = {"m": OP.zeros_like_state(ref), "v": OP.zeros_like_state(ref)}
    g = _random_grads(ref, seed=21, std=std)
    _upload_grads(st.opt, g)
    step = 7
    raw_ref = OP.grad_norm(g)
    scale = OP.combined_scale(raw_ref, tc)
    assert (scale != F32(1.0) / F32(2560.0)) == clipped
    raw_ref2 = OP.optimizer_step(ref, g, mom, step, tc)
    raw_dev = st.opt.step(step)
    print(f"norm device {raw_dev:.7e} oracle {raw_ref2:.7e} scale {scale:.4e}", flush=True)
    assert abs(raw_dev - raw_ref2) <= 1e-6 * raw_ref2
    dev = _device_state(st.opt, 0, cfg.nlayers)
    for a, b in [(dev["embed"], ref["embed"]), (dev["gamma_final"], ref["gamma_final"])] + \
            [(dl[kk], rl[kk]) for dl, rl in zip(dev["layers"], ref["layers"]) for kk in OP.LAYER_TENSORS]:
        np.testing.assert_allclose(a, b, rtol=2e-6, atol=1e-9)


def test_grad_norm_clip_and_zero(tiny_opt):
    cfg, k, w, st = tiny_opt
    ref = _state_of(w)
    g = _random_grads(ref, seed=31, std=0.5)
    _upload_grads(st.opt, g)
    n_ref = OP.grad_norm(g)
    assert abs(st.opt.grad_norm() - n_ref) <= 1e-6 * n_ref
    max_norm = float(n_ref) / 3
    assert abs(st.opt.clip_grads(max_norm) - n_ref) <= 1e-6 * n_ref
    OP.clip_grads(g, max_norm)
    dev = _device_state(st.opt, 3, cfg.nlayers)
    np.testing.assert_allclose(dev["embed"], g["embed"], rtol=1e-6)
    np.testing.assert_allclose(dev["layers"][1]["w2"], g["layers"][1]["w2"], rtol=1e-6)
    assert abs(st.opt.grad_norm() - max_norm) <= 1e-5 * max_norm
    ptr, n = st.opt.grad_arena()
    c = cfg
    per_layer = c.dim * (c.q_dim + 2 * c.kv_dim) + c.q_dim * c.dim + 3 * c.dim * c.hidden + 2 * c.dim
    assert ptr and n == c.nlayers * per_layer + c.vocab * c.dim + c.dim
    st.opt.zero_grads()
    assert st.opt.grad_norm() == 0.0


def test_forward_and_decode_use_updated_weights(tiny_opt):
    """After updates, the fp16 weights the GEMMs read (and the decode copy)
    equal the new master weights rounded to fp16."""
    cfg, k, w, st = tiny_opt
    tc = E.TrainConfig(max_lr=0.005, warmup_steps=1, total_steps=10)  # visible moves
    st.opt.close()
    st.opt = hb.Optimizer(k.model, tc)
    for l, lw in enumerate(w.layers):
        st.opt.upload_layer(l, lw)
    st.opt.upload_embed(w.embed, w.gamma_final)
    tok = tokens_for(cfg, cfg.seq + 1, seed=5)
    before = E.forward_logits(cfg, k, None, tok[:-1], tok[1:]).logits
    ref = _state_of(w)
    for s in range(3):
        _upload_grads(st.opt, _random_grads(ref, seed=40 + s, std=1.0))
        st.opt.step(s, want_norm=False)
    after = E.forward_logits(cfg, k, None, tok[:-1], tok[1:])
    dev = _device_state(st.opt, 0, cfg.nlayers)
    ow = O.ModelW(embed=f16_round(dev["embed"]), gamma_final=dev["gamma_final"],
                  layers=[O.LayerW(**{kk: (f16_round(lw[kk]) if kk.startswith("w") else lw[kk])
                                      for kk in O.LayerW.__dataclass_fields__}) for lw in dev["layers"]])
    r = O.model_forward(oracle_cfg(cfg), ow, tok[:-1], tok[1:])
    moved = np.abs(after.logits.reshape(-1) - before.reshape(-1)).max()
    err = np.abs(after.logits.reshape(-1) - r["logits"].reshape(-1)).max()
    print(f"logits moved by {moved:.3e}; vs oracle on the new weights {err:.3e}", flush=True)
    assert moved > 1e-2
    assert err < 2e-3
    np.testing.assert_allclose(after.losses, r["losses"], rtol=1e-3)
    dec = E.Decoder(k, batch=1, ctx_max=cfg.seq)
    gl, _ = dec.prefill(tok[:20])
    assert np.abs(gl[0] - after.logits.reshape(cfg.seq, cfg.vocab)[19]).max() < 2e-3
    gl, _ = dec.step([tok[20]])
    assert np.abs(gl[0] - after.logits.reshape(cfg.seq, cfg.vocab)[20]).max() < 2e-3


def test_large_tensors_bit_exact(gpu):
    """The 48M shape: the 16.4M-element embedding and the 0.8M-element
    matrices take several grid-stride passes of the AdamW kernel."""
    cfg = ModelConfig.llama_48m()
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=4, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        tc = OP.TrainConfig()
        ref = _state_of(w)
        mom = {"m": OP.zeros_like_state(ref), "v": OP.zeros_like_state(ref)}
        for t in (1, 2):
            g = _random_grads(ref, seed=50 + t, std=3e-3)
            _upload_grads(st.opt, g)
            OP.update_weights(ref, g, mom, t, F32(2e-4), tc, 1.0)
            st.opt.update_weights(t, 2e-4, 1.0)
        _assert_state_equal(_device_state(st.opt, 0, cfg.nlayers), ref, "weights")
        _assert_state_equal(_device_state(st.opt, 2, cfg.nlayers), mom["v"], "v")
    finally:
        st.close()


def test_synthetic_master_matches_host_values(gpu):
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    opt = hb.Optimizer(k.model, E.TrainConfig())
    try:
        opt.init_synthetic(77, 0.02)
        w = ModelWeights.synthetic(cfg, seed=77, std=0.02)
        dev = _device_state(opt, 0, cfg.nlayers)
        _assert_state_equal(dev, _state_of(w), "synthetic master")
        # and the model's fp16 weights are the same values rounded
        k._uploaded = ("synthetic", 77, 0.02)
        tok = tokens_for(cfg, cfg.seq + 1, seed=6)
        a = E.forward_logits(cfg, k, None, tok[:-1], tok[1:]).logits
        k2 = CompiledKernels.compile(cfg)
        b = E.forward_logits(cfg, k2, w, tok[:-1], tok[1:]).logits
        np.testing.assert_array_equal(a, b)
    finally:
        opt.close()


def test_optimizer_error_paths(gpu):
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    with pytest.raises(hb.HipBridgeError) as e:
        hb.Optimizer(k.model, E.TrainConfig(warmup_steps=0))
    assert e.value.code == hb.HB_E_INVALID
    opt = hb.Optimizer(k.model, E.TrainConfig())
    try:
        with pytest.raises(hb.HipBridgeError) as e:
            opt.update_weights(0, 1e-3, 1.0)  # t is 1-based
        assert e.value.code == hb.HB_E_INVALID
        with pytest.raises(hb.HipBridgeError):
            opt.download_layer(0, which=7)
        with pytest.raises(hb.HipBridgeError):
            opt.download_layer(cfg.nlayers, which=0)
        with pytest.raises(hb.HipBridgeError):
            opt.clip_grads(-1.0)
    finally:
        opt.close()
