"""RSTK checkpoints through the C ABI on the GPU: loading reproduces a direct
upload bit for bit, and saving writes exactly the oracle's bytes."""
import numpy as np
import pytest

import oracle.checkpoint as CK
from rustane_amd import engine as E
from rustane_amd import hip_bridge as hb
from rustane_amd.engine import CompiledKernels, ModelWeights
from tests._util import f16_round, oracle_weights, tiny_config, tokens_for

pytestmark = pytest.mark.gpu


def test_load_equals_direct_upload(gpu, tmp_path):
    cfg = tiny_config()
    w = ModelWeights.synthetic(cfg, seed=11, std=0.02)
    p = tmp_path / "ckpt_000005.bin"
    CK.write_rstk(p, cfg, oracle_weights(w), 5)
    k1 = CompiledKernels.compile(cfg)
    assert E.load_checkpoint(p, k1) == 5
    k2 = CompiledKernels.compile(cfg)
    tok = tokens_for(cfg, cfg.seq + 1, seed=12)
    a = E.forward_logits(cfg, k1, None, tok[:-1], tok[1:])
    b = E.forward_logits(cfg, k2, w, tok[:-1], tok[1:])
    np.testing.assert_array_equal(a.logits, b.logits)
    np.testing.assert_array_equal(a.losses, b.losses)


def test_save_from_model_and_from_optimizer_match_oracle_bytes(gpu, tmp_path):
    cfg = tiny_config()
    w = ModelWeights.synthetic(cfg, seed=13, std=0.02)
    ow = oracle_weights(w)
    # fp16-exact weights: the model's fp16 copy then holds them without loss
    for lw in ow.layers:
        for name in ("wq", "wk", "wv", "wo", "w1", "w3", "w2"):
            setattr(lw, name, f16_round(getattr(lw, name)))
    ow.embed = f16_round(ow.embed)
    k = CompiledKernels.compile(cfg)
    wex = ModelWeights(embed=ow.embed, gamma_final=ow.gamma_final,
                       layers=[E.LayerWeights(**{n: getattr(lw, n) for n in CK.LAYER_ORDER}) for lw in ow.layers])
    k.ensure_weights(wex)
    path = E.save_checkpoint(cfg, k, None, 9, tmp_path)
    assert path.endswith("ckpt_000009.bin")
    assert open(path, "rb").read() == CK.rstk_bytes(cfg, ow, 9)
    # from the optimizer: the unrounded fp32 master weights
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        p2 = E.save_checkpoint(cfg, k, st, 10, tmp_path / "opt")
        assert open(p2, "rb").read() == CK.rstk_bytes(cfg, oracle_weights(w), 10)
        # and loading it back into a fresh optimizer restores the master copy
        k3 = CompiledKernels.compile(cfg)
        st3 = E.ModelOptState(k3, E.TrainConfig())
        assert E.load_checkpoint(p2, k3, st3) == 10
        lw = st3.opt.download_layer(1, 0)
        np.testing.assert_array_equal(lw["w2"], w.layers[1].w2)
        e, g = st3.opt.download_embed(0)
        np.testing.assert_array_equal(e, w.embed)
        st3.close()
    finally:
        st.close()


def test_load_rejects_mismatched_files(gpu, tmp_path):
    cfg = tiny_config()
    w = ModelWeights.synthetic(cfg, seed=14, std=0.02)
    p = tmp_path / "a.bin"
    CK.write_rstk(p, cfg, oracle_weights(w), 1)
    other = tiny_config(dim=192)
    k = CompiledKernels.compile(other)
    with pytest.raises(hb.HipBridgeError) as e:
        E.load_checkpoint(p, k)
    assert e.value.code == hb.HB_E_CONFIG
    k2 = CompiledKernels.compile(cfg)
    cut = tmp_path / "cut.bin"
    cut.write_bytes(p.read_bytes()[:-4])
    with pytest.raises(hb.HipBridgeError) as e:
        E.load_checkpoint(cut, k2)
    assert e.value.code == hb.HB_E_INVALID
    with pytest.raises(hb.HipBridgeError) as e:  # nothing uploaded yet: nothing to save
        hb.rstk_save(k2.model, tmp_path / "x.bin", 1)
    assert e.value.code == hb.HB_E_STATE
