"""Validation on the GPU (hb_validate: bin/train.rs:123-163 with the token
stream resident on the device) against the oracle, and against the
reference's host loop run on the same device forward."""
import numpy as np
import pytest

import oracle.data as OD
from rustane_amd import engine as E
from rustane_amd import hip_bridge as hb
from rustane_amd.engine import CompiledKernels, ModelWeights
from tests._util import oracle_cfg, oracle_weights, tiny_config

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup(gpu, tmp_path_factory):
    cfg = tiny_config()
    w = ModelWeights.synthetic(cfg, seed=21, std=0.02)
    k = CompiledKernels.compile(cfg)
    k.ensure_weights(w)
    rng = np.random.default_rng(7)
    d = tmp_path_factory.mktemp("data")
    toks = rng.integers(0, cfg.vocab, 1000).astype("<u2")
    toks.tofile(d / "val.bin")
    tb = rng.integers(0, 5, cfg.vocab).astype("<i4")  # about a fifth are special (0 bytes)
    tb.tofile(d / "token_bytes.bin")
    return cfg, w, k, E.TokenData.open(d / "val.bin"), E.TokenBytes.load(d / "token_bytes.bin"), d


def test_validate_matches_oracle_and_host_loop(setup):
    cfg, w, k, td, tb, _ = setup
    steps = 30  # wraps around the 1000-token stream (max_pos 959)
    avg, bpb = E.validate(cfg, k, w, td, tb, steps)
    ra, rb, rn, rbytes = OD.validate(oracle_cfg(cfg), oracle_weights(w), np.asarray(td._t), tb.bytes, steps)
    ha, hbpb = E.validate_host(cfg, k, w, td, tb, steps)
    print(f"device avg {avg:.6f} bpb {bpb:.6f} | host loop {ha:.6f} {hbpb:.6f} | oracle {ra:.6f} {rb:.6f}",
          flush=True)
    assert abs(avg - ra) <= 1e-3 * ra and abs(bpb - rb) <= 1e-3 * rb
    assert abs(avg - ha) <= 2e-6 * ha and abs(bpb - hbpb) <= 2e-6 * hbpb
    _, _, nats, nbytes = hb.validate(k.model, td.device(k), tb.bytes, steps)
    assert nbytes == rbytes and abs(nats - rn) <= 1e-3 * rn


def test_batched_windows_agree(setup):
    cfg, w, k, td, tb, _ = setup
    a1, b1, n1, y1 = hb.validate(k.model, td.device(k), tb.bytes, 12, 1)
    a4, b4, n4, y4 = hb.validate(k.model, td.device(k), tb.bytes, 12, 4)
    a5, b5, _, _ = hb.validate(k.model, td.device(k), tb.bytes, 12, 5)  # a short last group
    assert y1 == y4
    for x, y in ((a1, a4), (b1, b4), (a1, a5), (b1, b5)):
        assert abs(x - y) <= 1e-5 * abs(x)
    a0, b0, _, y0 = hb.validate(k.model, td.device(k), None, 12, 4)
    assert abs(a0 - a4) <= 1e-6 * a4 and b0 == 0.0 and y0 == 0


def test_validate_errors(setup):
    cfg, w, k, td, tb, d = setup
    short = hb.DeviceTokens(k.ctx, tokens=np.arange(cfg.seq + 1, dtype="<u2"))
    with pytest.raises(hb.HipBridgeError) as e:
        hb.validate(k.model, short, None, 1)
    assert e.value.code == hb.HB_E_INVALID
    bad = np.zeros(500, "<u2")
    bad[100] = cfg.vocab  # outside the vocabulary
    badt = hb.DeviceTokens(k.ctx, tokens=bad)
    with pytest.raises(hb.HipBridgeError) as e:
        hb.validate(k.model, badt, None, 5)
    assert e.value.code == hb.HB_E_INVALID
    # the error word is cleared: the next call works
    hb.validate(k.model, td.device(k), None, 2)
    (d / "odd.bin").write_bytes(b"\x01\x02\x03")
    with pytest.raises(hb.HipBridgeError):
        hb.DeviceTokens(k.ctx, path=d / "odd.bin")
    opened = hb.DeviceTokens(k.ctx, path=d / "val.bin")
    assert len(opened) == td.len()
