"""RSTK checkpoint format of bin/train.rs:165-202 (TEST INFRASTRUCTURE ONLY).

save_checkpoint writes: b"RSTK", then little-endian u32 version (1), step,
dim, nlayers, vocab, seq (train.rs:175-183), then fp32 little-endian values
(write_f32_vec, train.rs:199-202) of embed, gamma_final and, per layer, wq,
wk, wv, wo, w1, w3, w2, gamma1, gamma2 (train.rs:186-192), each in its
LayerWeights/ModelWeights layout. Pins: tests/test_checkpoint_oracle.py.
"""
from __future__ import annotations

import struct

import numpy as np

from .forward import LayerW, ModelW

LAYER_ORDER = ("wq", "wk", "wv", "wo", "w1", "w3", "w2", "gamma1", "gamma2")


def rstk_bytes(cfg, weights: ModelW, step: int) -> bytes:
    """train.rs:172-196 as one byte string."""
    out = [b"RSTK", struct.pack("<6I", 1, step, cfg.dim, cfg.nlayers, cfg.vocab, cfg.seq)]
    out.append(np.asarray(weights.embed, "<f4").tobytes())
    out.append(np.asarray(weights.gamma_final, "<f4").tobytes())
    for lw in weights.layers:
        for name in LAYER_ORDER:
            out.append(np.asarray(getattr(lw, name), "<f4").tobytes())
    return b"".join(out)


def write_rstk(path, cfg, weights: ModelW, step: int) -> None:
    with open(path, "wb") as f:
        f.write(rstk_bytes(cfg, weights, step))


def read_rstk(path, cfg):
    """Inverse of rstk_bytes for a config whose hidden/q/kv sizes the header
    does not carry; returns (header dict, ModelW)."""
    data = open(path, "rb").read()
    if data[:4] != b"RSTK":
        raise ValueError("bad magic")
    version, step, dim, nl, vocab, seq = struct.unpack_from("<6I", data, 4)
    if version != 1:
        raise ValueError("bad version")
    f = np.frombuffer(data, "<f4", offset=28)
    d, q, kv, h = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden
    sizes = dict(wq=d * q, wk=d * kv, wv=d * kv, wo=q * d, w1=d * h, w3=d * h, w2=d * h,
                 gamma1=d, gamma2=d)
    o = 0

    def take(n):
        nonlocal o
        a = f[o:o + n].astype(np.float32)
        o += n
        return a

    embed = take(vocab * dim)
    gamma_final = take(dim)
    layers = [LayerW(**{name: take(sizes[name]) for name in LAYER_ORDER}) for _ in range(nl)]
    if o != f.size:
        raise ValueError("size does not match the config")
    hdr = dict(version=version, step=step, dim=dim, nlayers=nl, vocab=vocab, seq=seq)
    return hdr, ModelW(embed=embed, layers=layers, gamma_final=gamma_final)
