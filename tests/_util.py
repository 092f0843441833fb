"""Shared helpers for the tests (not collected: no test_ prefix)."""
import numpy as np

from rustane_amd.engine import ModelConfig, ModelWeights

F32 = np.float32


def tiny_config(**kw) -> ModelConfig:
    """Smallest shape the library accepts (dims multiple of 64, hd 64); seq 40 is
    deliberately not a multiple of 32 so attention padding is exercised."""
    base = dict(dim=128, hidden=256, heads=2, nlayers=2, seq=40, vocab=256, hd=64)
    base.update(kw)
    return ModelConfig.make(**base)


def oracle_cfg(cfg):
    import oracle as O
    return O.Config.of(cfg)


def oracle_weights(w: ModelWeights):
    import oracle as O
    return O.ModelW.of(w)


def to_dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def f16_round(a):
    return np.asarray(a, F32).astype(np.float16).astype(F32)


def tokens_for(cfg, n, seed=42, stream=0):
    from rustane_amd import hip_bridge as hb
    return hb.synth_tokens(seed, stream, cfg.vocab, n)
