#!/usr/bin/env python3
"""Precision floor of fp16 GEMM operands, attributed per rounding point
(a study script, not a test; CPU only).

Runs the oracle's forward arithmetic (token-major, fp32) on the weights the
device holds (fp16-rounded, kept as fp32), once per *variant*. A variant says,
for each point where the device's kernels narrow an operand, whether that
operand is kept in fp32 ("32"), rounded to fp16 ("16", what a plain fp16 MFMA
operand does), or split into an fp16 pair hi + lo with lo = fp16(x - hi) ("2",
what a kernel that runs two MFMAs per k-step on that operand computes). The
rounding points, in forward order:

  xn    normalised rows fed to the QKV GEMM
  q, k  Q and K after RoPE (the attention score product)
  v     V (the P.V product)
  p     attention probabilities (the P.V product)
  attn  attention output fed to the Wo GEMM
  x2n   normalised rows fed to the W1|W3 GEMM
  gate  SwiGLU gate fed to the W2 GEMM
  xf    final normalised rows fed to the logits GEMM

Every variant is compared with the all-fp32 variant on the same weights and
tokens: max |dlogit|, rms dlogit, max relative per-position loss error and
greedy top-1 agreement. All variants advance through the layers together, so
each layer's weights are generated once.

  python tests/fp16_emulation_study.py 7b              attribution table, seed 46 (~15 min on 8 cores)
  python tests/fp16_emulation_study.py 600m
  python tests/fp16_emulation_study.py 7b --variants "all;all,xf=2;all,q=2,k=2"

Variant syntax: tokens separated by ',' applied left to right, the last one
that covers a (point, layer) wins; "all" / "fp32" set every point to 16 / 32,
"<point>=<16|2|32>" sets one point, "<point>@a:b=<mode>" sets it in layers
a..b-1 only, "*" stands for every point; xf counts as layer nlayers. Points
no token covers stay fp32. Default: fp32, all, each point alone, all but each
point. With --vs-unrounded the weights may differ too: "w@a:b=32" keeps the
unrounded fp32 weights of layers a..b-1, "e=32" the embedding rows the input
gathers, "elog=32" the embedding in the logits product (fp16 otherwise, as
the device holds them); every variant is then compared with fp32 arithmetic
on the unrounded weights.

Inputs: the first sequence of tokens_for(cfg, S + 1, seed) (the same draw as
the full-size tests), seq 512, synthetic N(0, 0.02) weights of seed 1234.
"""
import argparse
import os
import sys
import time

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import oracle as O  # noqa: E402
from rustane_amd.engine import ModelConfig  # noqa: E402
from tests._util import synthetic_oracle_weights, tokens_for  # noqa: E402

F32 = np.float32
POINTS = ("xn", "q", "k", "v", "p", "attn", "x2n", "gate", "xf")


def r16(a):
    return np.asarray(a, F32).astype(np.float16).astype(F32)


def r2x16(a):
    a = np.asarray(a, F32)
    hi = r16(a)
    return hi + r16(a - hi)


ROUND = {"32": lambda a: a, "16": r16, "2": r2x16}


WEIGHT_POINTS = ("w", "e", "elog")  # layer weights, embedding rows gathered, embedding in the logits


def parse_variant(spec):
    """-> {point: [(first layer, end layer, mode), ...]}; the last matching rule wins.
    Weight points (w, e, elog) default to 16 (the device's fp16 weights); "=32"
    uses the unrounded fp32 values (run() then needs unrounded weights)."""
    rules = {p: [] for p in POINTS + WEIGHT_POINTS}
    inf = 1 << 30
    for tok in filter(None, (t.strip() for t in spec.split(","))):
        if tok in ("all", "fp32"):
            for p in POINTS:
                rules[p] = [(0, inf, "16" if tok == "all" else "32")]
            continue
        lhs, _, mode = tok.partition("=")
        pt, _, rng = lhs.partition("@")
        a, _, b = rng.partition(":")
        lo, hi = (int(a or 0), int(b) if b else inf) if rng else (0, inf)
        if pt not in POINTS + WEIGHT_POINTS + ("*",) or mode not in ROUND:
            raise SystemExit(f"bad variant token {tok!r}")
        for p in (POINTS if pt == "*" else (pt,)):
            rules[p].append((lo, hi, mode))
    for p in WEIGHT_POINTS:
        rules[p] = [(0, inf, "16")] + rules[p]
    return rules


def default_variants():
    out = ["fp32", "all"]
    out += [f"{p}=16" for p in POINTS]
    out += [f"all,{p}=32" for p in POINTS]
    return out


class Stream:
    """One variant's residual stream."""

    def __init__(self, spec):
        self.spec = spec
        self.rules = parse_variant(spec)
        self.x = None

    def at(self, layer):
        """{point: rounding function} in this layer (the final norm counts as layer nlayers)."""
        out = {}
        for p, rl in self.rules.items():
            if p in WEIGHT_POINTS:
                out[p] = [m for lo, hi, m in rl if lo <= layer < hi][-1]
                continue
            mode = "32"
            for lo, hi, m in rl:
                if lo <= layer < hi:
                    mode = m
            out[p] = ROUND[mode]
        return out


def run(cfg, ow, tok, S, specs, log_every=8, unrounded=False):
    """Logits and per-position losses of each variant. unrounded: ow holds the
    unrounded fp32 weights (the weight points then choose per variant)."""
    d, H, hd, q, hid = cfg.dim, cfg.heads, cfg.hd, cfg.q_dim, cfg.hidden
    KVH, kv = cfg.kv_heads, cfg.kv_dim
    rep = H // KVH
    cos, sin = O.rope_table(S, hd)
    alpha = O.Config.of(cfg).alpha()
    mask = np.triu(np.full((S, S), -np.inf, F32), 1)
    sc_scale = F32(1.0) / np.sqrt(F32(hd))

    def norm(x, g):
        ss = (x * x).sum(1, dtype=F32, keepdims=True)
        return x * (F32(1) / np.sqrt(ss * F32(1.0 / d) + F32(1e-5))) * g

    def rope(a):
        a = a.reshape(S, -1, hd)
        rot = np.empty_like(a)
        rot[..., 0::2] = -a[..., 1::2]
        rot[..., 1::2] = a[..., 0::2]
        return (a * cos[:, None] + rot * sin[:, None]).reshape(S, -1)

    # ow holds the device's fp16-rounded weights, or the unrounded ones when a
    # variant asks for fp32 weights somewhere (then each variant rounds itself)
    E32 = ow.embed.reshape(-1, d)
    E16 = r16(E32) if unrounded else E32
    streams = [Stream(s) for s in specs]
    for st in streams:
        st.x = (E32 if st.at(0)["e"] == "32" else E16)[tok[:-1]].astype(F32)
    t0 = time.time()
    for l in range(cfg.nlayers):
        lw = ow.layers[l]
        w32 = (lw.wq.reshape(d, q), lw.wk.reshape(d, kv), lw.wv.reshape(d, kv), lw.wo.reshape(q, d),
               lw.w1.reshape(d, hid), lw.w3.reshape(d, hid), lw.w2.reshape(d, hid).T)
        w16 = tuple(r16(a) for a in w32) if unrounded else w32
        for st in streams:
            R, x = st.at(l), st.x
            wq, wk, wv, wo, w1, w3, w2t = w32 if R["w"] == "32" else w16
            xn = R["xn"](norm(x, lw.gamma1))
            Q = R["q"](rope(xn @ wq))
            K = R["k"](rope(xn @ wk))
            V = R["v"](xn @ wv)
            q4 = Q.reshape(S, H, hd).transpose(1, 0, 2)
            k4 = np.repeat(K.reshape(S, KVH, hd).transpose(1, 0, 2), rep, axis=0)
            v4 = np.repeat(V.reshape(S, KVH, hd).transpose(1, 0, 2), rep, axis=0)
            sc = np.matmul(q4, k4.transpose(0, 2, 1)) * sc_scale + mask
            p = np.exp(sc - sc.max(-1, keepdims=True))
            a = (np.matmul(R["p"](p), v4) / p.sum(-1, keepdims=True)).transpose(1, 0, 2).reshape(S, q)
            x2 = x + alpha * (R["attn"](a) @ wo)
            x2n = R["x2n"](norm(x2, lw.gamma2))
            h1 = x2n @ w1
            h3 = x2n @ w3
            g = R["gate"](h1 / (F32(1) + np.exp(-h1)) * h3)
            st.x = x2 + alpha * (g @ w2t)
        if (l + 1) % log_every == 0:
            print(f"  layer {l + 1}/{cfg.nlayers} ({time.time() - t0:.0f} s)", flush=True)
    out = []
    for st in streams:
        R = st.at(cfg.nlayers)
        lg = R["xf"](norm(st.x, ow.gamma_final)) @ (E32 if R["elog"] == "32" else E16).T
        m = lg.max(1, keepdims=True)
        lse = np.log(np.exp(lg - m).sum(1)) + m[:, 0]
        out.append((lg, lse - lg[np.arange(S), tok[1:]]))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("shape", choices=["600m", "5b", "7b"])
    ap.add_argument("--seed", type=int, default=None)
    ap.add_argument("--seq", type=int, default=512)
    ap.add_argument("--variants", default=None, help="';'-separated variant specs")
    ap.add_argument("--vs-unrounded", action="store_true",
                    help="compare with fp32 arithmetic on the unrounded fp32 weights instead "
                         "(adds the weights' own fp16 rounding to every variant)")
    a = ap.parse_args()
    seed = a.seed if a.seed is not None else {"7b": 46, "5b": 44}.get(a.shape, 42)
    cfg = {"7b": ModelConfig.llama_7b(), "5b": ModelConfig.llama_5b(),
           "600m": ModelConfig.llama_600m()}[a.shape]
    specs = a.variants.split(";") if a.variants else default_variants()
    if "fp32" not in specs:
        specs = ["fp32"] + specs
    S = a.seq
    tok = tokens_for(cfg, S + 1, seed=seed)
    t0 = time.time()
    if a.vs_unrounded:
        ow = synthetic_oracle_weights(cfg, 1234, round16=False, cache=False)
        ref = "fp32,w=32,e=32,elog=32"
        res = dict(zip(specs + [ref], run(cfg, ow, tok, S, specs + [ref], unrounded=True)))
        L0, l0 = res[ref]
        against = "fp32 arithmetic on the unrounded fp32 weights"
    else:
        ow = synthetic_oracle_weights(cfg, 1234, round16=True, cache=False)
        res = dict(zip(specs, run(cfg, ow, tok, S, specs)))
        L0, l0 = res["fp32"]
        against = "all-fp32 operands on the device's weights"
    print(f"{a.shape} seq {S} seed {seed}: each variant vs {against} ({time.time() - t0:.0f} s)")
    print(f"{'variant':<24} {'max|dlogit|':>11} {'rms dlogit':>10} {'max rel dloss':>13} {'top-1':>7}")
    for s in dict.fromkeys(specs):
        if s == "fp32" and not a.vs_unrounded:
            continue
        L1, l1 = res[s]
        dl = L1 - L0
        print(f"{s:<24} {np.abs(dl).max():>11.3e} {np.sqrt((dl * dl).mean()):>10.3e} "
              f"{(np.abs(l1 - l0) / l0).max():>13.3e} {(L1.argmax(1) == L0.argmax(1)).mean():>7.4f}",
              flush=True)


if __name__ == "__main__":
    main()
