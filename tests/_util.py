"""Shared helpers for the tests (not collected: no test_ prefix)."""
import numpy as np

from rustane_amd.engine import ModelConfig, ModelWeights

F32 = np.float32

# Parity comparisons of this pytest run (label, max |dlogit|, max rel dloss,
# agreeing and compared top-1 positions, whether against the oracle); printed
# by conftest.py's terminal summary.
PARITY = []


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


class SyntheticLayers:
    """Oracle LayerW for every layer, generated on first access from the seeded
    stream that hb_model_init_synthetic writes on the device (tensor ids
    16*layer + 0..6, gammas 1), so a full-size oracle never needs a device
    copy. cache=True keeps each generated layer (7B: 26.4 GB of fp32 in all)."""

    def __init__(self, cfg, seed, std=0.02, cache=True, round16=False):
        self.cfg, self.seed, self.std, self.cache, self.round16 = cfg, seed, std, cache, round16
        self._layers = {}

    def __len__(self):
        return self.cfg.nlayers

    def __getitem__(self, l):
        import oracle as O
        from rustane_amd.engine import LayerWeights
        if not 0 <= l < self.cfg.nlayers:
            raise IndexError(l)
        if l in self._layers:
            return self._layers[l]
        lw = LayerWeights.synthetic(self.cfg, l, self.seed, self.std)
        ow = O.LayerW(**{k: f16_round(getattr(lw, k)) if self.round16 else getattr(lw, k)
                         for k in O.LayerW.__dataclass_fields__})
        if self.cache:
            self._layers[l] = ow
        return ow

    def __iter__(self):
        return (self[l] for l in range(len(self)))


def synthetic_oracle_weights(cfg, seed, std=0.02, cache=True, round16=False):
    """O.ModelW equal to ModelWeights.synthetic(cfg, seed, std), layers generated lazily.
    round16=True rounds every weight to fp16 (the values the device holds) and
    keeps them as fp32 for the oracle's arithmetic."""
    import oracle as O
    from rustane_amd import hip_bridge as hb
    e = hb.synth_normal(seed, hb.HB_SYNTH_EMBED_ID, cfg.vocab * cfg.dim, std)
    return O.ModelW(embed=f16_round(e) if round16 else e,
                    layers=SyntheticLayers(cfg, seed, std, cache, round16),
                    gamma_final=np.ones(cfg.dim, F32))
