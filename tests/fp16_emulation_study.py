#!/usr/bin/env python3
"""Precision floor of fp16 GEMM inputs (a study script, not a test; CPU only).

Runs the oracle's forward twice on the weights the device holds (fp16-rounded,
kept as fp32): once in plain fp32, once rounding to fp16 exactly where the
device's kernels do -- the normalised rows fed to the QKV and W1|W3 GEMMs, Q/K
after RoPE and V, the attention probabilities fed to the P.V product, the
attention output, the SwiGLU gate and the final normalised rows fed to the
logits GEMM -- and prints the max |dlogit|, max relative per-position loss
error and top-1 agreement between the two. That is the error any kernel that
feeds fp16 operands to MFMA starts from; tests/test_gpu_fullsize.py quotes it.

  python tests/fp16_emulation_study.py 7b [seed]      (~7 min on 8 cores)
  python tests/fp16_emulation_study.py 600m [seed]

Inputs: the first sequence of tokens_for(cfg, 513, seed) (the same draw as the
full-size tests), seq 512, synthetic N(0, 0.02) weights of seed 1234.
"""
import os
import sys
import time

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import oracle as O  # noqa: E402
from rustane_amd.engine import ModelConfig  # noqa: E402
from tests._util import synthetic_oracle_weights, tokens_for  # noqa: E402

F32 = np.float32


def r16(a):
    return np.asarray(a, F32).astype(np.float16).astype(F32)


def forward(cfg, ow, tok, S, emulate):
    """Token-major restatement of oracle.model_forward (same arithmetic in fp32),
    with fp16 rounding at the device's rounding points when emulate is set."""
    R = r16 if emulate else (lambda a: a)
    d, H, hd, q, hid = cfg.dim, cfg.heads, cfg.hd, cfg.q_dim, cfg.hidden
    cos, sin = O.rope_table(S, hd)
    alpha = O.Config.of(cfg).alpha()

    def norm(x, g):
        ss = (x * x).sum(1, dtype=F32, keepdims=True)
        return x * (F32(1) / np.sqrt(ss * F32(1.0 / d) + F32(1e-5))) * g

    def rope(a):
        a = a.reshape(S, -1, hd)
        rot = np.empty_like(a)
        rot[..., 0::2] = -a[..., 1::2]
        rot[..., 1::2] = a[..., 0::2]
        return (a * cos[:, None] + rot * sin[:, None]).reshape(S, -1)

    E = ow.embed.reshape(-1, d)
    x = E[tok[:-1]].astype(F32)
    mask = np.triu(np.full((S, S), -np.inf, F32), 1)
    for l in range(cfg.nlayers):
        lw = ow.layers[l]
        xn = R(norm(x, lw.gamma1))
        Q = R(rope(xn @ lw.wq.reshape(d, q)))
        K = R(rope(xn @ lw.wk.reshape(d, q)))
        V = R(xn @ lw.wv.reshape(d, q))
        q4, k4, v4 = (t.reshape(S, H, hd).transpose(1, 0, 2) for t in (Q, K, V))
        sc = (q4 @ k4.transpose(0, 2, 1)) * F32(1 / np.sqrt(hd)) + mask
        p = np.exp(sc - sc.max(-1, keepdims=True))
        a = R(((R(p) @ v4) / p.sum(-1, keepdims=True)).transpose(1, 0, 2).reshape(S, q))
        x2 = x + alpha * (a @ lw.wo.reshape(q, d))
        x2n = R(norm(x2, lw.gamma2))
        h1 = x2n @ lw.w1.reshape(d, hid)
        h3 = x2n @ lw.w3.reshape(d, hid)
        g = R(h1 / (1 + np.exp(-h1)) * h3)
        x = x2 + alpha * (g @ lw.w2.reshape(d, hid).T)
    lg = R(norm(x, ow.gamma_final)) @ E.T
    m = lg.max(1, keepdims=True)
    lse = np.log(np.exp(lg - m).sum(1)) + m[:, 0]
    return lg, lse - lg[np.arange(S), tok[1:]]


def main():
    name = sys.argv[1] if len(sys.argv) > 1 else "600m"
    seed = int(sys.argv[2]) if len(sys.argv) > 2 else {"7b": 46, "5b": 44}.get(name, 42)
    cfg = {"7b": ModelConfig.llama_7b(), "5b": ModelConfig.llama_5b(),
           "600m": ModelConfig.llama_600m()}[name]
    ow = synthetic_oracle_weights(cfg, 1234, round16=True, cache=(name == "600m"))
    S = 512
    tok = tokens_for(cfg, S + 1, seed=seed)
    t0 = time.time()
    L0, l0 = forward(cfg, ow, tok, S, False)
    L1, l1 = forward(cfg, ow, tok, S, True)
    print(f"{name} seed {seed}: fp16-input emulation vs fp32 on the device's weights: "
          f"max|dlogit| {np.abs(L1 - L0).max():.3e}  max rel dloss {(np.abs(l1 - l0) / l0).max():.3e}  "
          f"top-1 {(L1.argmax(1) == L0.argmax(1)).mean():.4f}  ({time.time() - t0:.0f} s)", flush=True)


if __name__ == "__main__":
    main()
