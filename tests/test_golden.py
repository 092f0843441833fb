"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces its committed outputs (a regression guard on
the oracle itself). GPU: the device path meets the parity bars against the
fixtures directly, without running the oracle on the GPU host.
"""
import os

import numpy as np
import pytest

import oracle as O
from tests.golden import make_golden as G

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", ["tiny", "llama48m"])
def test_oracle_reproduces_fixture(name):
    fx = load(name)
    cfg, w, tok = G.inputs(name)
    oc, ow = O.Config.of(cfg), O.ModelW.of(w)
    S = len(tok) - 1
    out = O.model_forward(oc, ow, tok[:-1], tok[1:])
    logits = out["logits"].reshape(S, cfg.vocab)
    np.testing.assert_allclose(out["losses"], fx["losses"], rtol=1e-5)
    np.testing.assert_allclose(logits[fx["logit_rows"]][:, :512], fx["logits_sub"], atol=1e-5)
    assert (logits.argmax(1) == fx["argmax"]).mean() >= 0.998


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tiny", "llama48m"])
def test_device_matches_fixture(gpu, name):
    from rustane_amd import engine as E
    fx = load(name)
    cfg, w, tok = G.inputs(name)
    k = E.CompiledKernels.compile(cfg)
    k.init_synthetic(G.CASES[name][2], G.STD)  # device-side generation of the same weights
    S = len(tok) - 1
    res = E.forward_logits(cfg, k, None, tok[:-1], tok[1:])
    logits = res.logits.reshape(S, cfg.vocab)
    rel = np.abs(res.losses - fx["losses"]) / fx["losses"]
    err = np.abs(logits[fx["logit_rows"]][:, :512] - fx["logits_sub"]).max()
    top1 = (logits.argmax(1) == fx["argmax"]).mean()
    print(f"{name}: max rel dloss {rel.max():.2e}, max |dlogit| (subset) {err:.2e}, top1 {top1:.4f}", flush=True)
    assert rel.max() < 1e-3
    assert err < 2e-2
    assert np.abs(logits.max(1) - fx["logit_rowmax"]).max() < 2e-2
    assert top1 >= 0.995
    # teacher-forced decode against the fixture's steps
    P = int(fx["decode_prefill"])
    dec = E.Decoder(k, batch=1, ctx_max=S)
    gl, _ = dec.prefill(tok[:P])
    got = [gl[0]]
    for p in range(P, P + len(fx["decode_argmax"]) - 1):
        gl, _ = dec.step([tok[p]])
        got.append(gl[0])
    got = np.stack(got)
    assert np.abs(got[:, :512] - fx["decode_logits_sub"]).max() < 2e-2
    assert (got.argmax(1) == fx["decode_argmax"]).mean() >= 6 / 7
