"""Writes the golden fixtures in this directory from the CPU oracle.

  python tests/golden/make_golden.py

Each fixture holds the inputs that define it (config, weight seed/std, token
seed) and the oracle's outputs. Weights and tokens come from the library's
seeded generators (hb_synth_normal / hb_synth_tokens), so a fixture is small:
only the expected outputs are stored.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402
from rustane_amd import engine as E  # noqa: E402
from rustane_amd import hip_bridge as hb  # noqa: E402

CASES = {
    # name: (config kwargs for ModelConfig.make, seq used, weight seed)
    "tiny": (dict(dim=128, hidden=256, heads=2, nlayers=2, seq=40, vocab=256, hd=64), 40, 1234),
    "llama48m": (dict(dim=512, hidden=1536, heads=8, nlayers=8, seq=512, vocab=32000, hd=64), 512, 1234),
}
STD = 0.02
TOKEN_SEED = 42


def config(name):
    kw, _, _ = CASES[name]
    return E.ModelConfig.make(**kw)


def inputs(name):
    kw, S, wseed = CASES[name]
    cfg = config(name)
    w = E.ModelWeights.synthetic(cfg, seed=wseed, std=STD)
    tok = hb.synth_tokens(TOKEN_SEED, 0, cfg.vocab, S + 1)
    return cfg, w, tok


def make(name):
    cfg, w, tok = inputs(name)
    oc, ow = O.Config.of(cfg), O.ModelW.of(w)
    S = len(tok) - 1
    out = O.model_forward(oc, ow, tok[:-1], tok[1:])
    logits = out["logits"].reshape(S, cfg.vocab)
    rows = np.unique(np.array([0, 1, S // 2, S - 1]))
    res = dict(losses=out["losses"], loss=np.float32(out["loss"]), argmax=logits.argmax(1).astype(np.int32),
               logit_rows=rows, logits_sub=logits[rows][:, :512].copy(),
               logit_rowmax=logits.max(1), logit_rowmean=logits.mean(1, dtype=np.float64).astype(np.float32))
    # teacher-forced decode: prefill P tokens then steps; last-position logits per step
    P = S // 2
    dec = O.DecodeOracle(oc, ow, ctx_max=S)
    steps = [dec.prefill(tok[:P])]
    for p in range(P, min(P + 6, S)):
        steps.append(dec.step(int(tok[p])))
    steps = np.stack(steps)
    res.update(decode_prefill=np.int32(P), decode_argmax=steps.argmax(1).astype(np.int32),
               decode_logits_sub=steps[:, :512].copy())
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **res)
    print(name, {k: getattr(v, "shape", v) for k, v in res.items()})


if __name__ == "__main__":
    for n in (sys.argv[1:] or CASES):
        make(n)
