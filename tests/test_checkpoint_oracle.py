"""RSTK checkpoint format (bin/train.rs:165-202): the oracle writer/reader and
the library's host-only header reader, no GPU needed."""
import os
import struct

import numpy as np
import pytest

import oracle as O
import oracle.checkpoint as CK
from rustane_amd import hip_bridge as hb
from tests._util import tiny_config


def _weights(cfg, seed=1):
    rng = np.random.default_rng(seed)
    n = lambda k: rng.standard_normal(k).astype(np.float32)
    d, q, kv, h = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden
    layers = [O.LayerW(wq=n(d * q), wk=n(d * kv), wv=n(d * kv), wo=n(q * d), w1=n(d * h), w3=n(d * h),
                       w2=n(d * h), gamma1=n(d), gamma2=n(d)) for _ in range(cfg.nlayers)]
    return O.ModelW(embed=n(cfg.vocab * d), layers=layers, gamma_final=n(d))


def test_round_trip_and_reference_size(tmp_path):
    cfg = tiny_config()
    w = _weights(cfg)
    p = tmp_path / "ckpt_000007.bin"
    CK.write_rstk(p, cfg, w, 7)
    # size from the reference's own parameter count (bin/train.rs:216-219)
    per_layer = (cfg.dim * cfg.q_dim + cfg.dim * cfg.kv_dim * 2 + cfg.q_dim * cfg.dim
                 + cfg.dim * cfg.hidden * 3 + cfg.dim * 2)
    total = cfg.vocab * cfg.dim + cfg.nlayers * per_layer + cfg.dim
    assert os.path.getsize(p) == 28 + 4 * total
    hdr, r = CK.read_rstk(p, cfg)
    assert hdr == dict(version=1, step=7, dim=cfg.dim, nlayers=cfg.nlayers, vocab=cfg.vocab, seq=cfg.seq)
    np.testing.assert_array_equal(r.embed, w.embed)
    np.testing.assert_array_equal(r.gamma_final, w.gamma_final)
    for a, b in zip(r.layers, w.layers):
        for k in CK.LAYER_ORDER:
            np.testing.assert_array_equal(getattr(a, k), getattr(b, k))


def test_write_order_follows_save_checkpoint(tmp_path):
    """Every tensor filled with its own constant: the values appear at the
    offsets train.rs:186-192's order gives (embed, gamma_final, then per layer
    wq wk wv wo w1 w3 w2 gamma1 gamma2)."""
    cfg = tiny_config()
    w = _weights(cfg)
    w.embed[:] = 1.0
    w.gamma_final[:] = 2.0
    for l, lw in enumerate(w.layers):
        for i, k in enumerate(CK.LAYER_ORDER):
            getattr(lw, k)[:] = 10 * (l + 1) + i
    data = CK.rstk_bytes(cfg, w, 3)
    assert data[:4] == b"RSTK" and struct.unpack_from("<6I", data, 4)[:2] == (1, 3)
    vals = np.frombuffer(data, "<f4", offset=28)
    runs, start = [], 0
    for i in range(1, vals.size + 1):
        if i == vals.size or vals[i] != vals[start]:
            runs.append((float(vals[start]), i - start))
            start = i
    d, q, kv, h = cfg.dim, cfg.q_dim, cfg.kv_dim, cfg.hidden
    sizes = [d * q, d * kv, d * kv, q * d, d * h, d * h, d * h, d, d]
    expect = [(1.0, cfg.vocab * d), (2.0, d)] + [(10.0 * (l + 1) + i, sizes[i])
                                                 for l in range(cfg.nlayers) for i in range(9)]
    assert runs == expect


def test_library_reads_the_header(tmp_path):
    cfg = tiny_config()
    p = tmp_path / "a.bin"
    CK.write_rstk(p, cfg, _weights(cfg), 123)
    assert hb.rstk_read_header(p) == dict(version=1, step=123, dim=cfg.dim, nlayers=cfg.nlayers,
                                          vocab=cfg.vocab, seq=cfg.seq)
    bad = tmp_path / "bad.bin"
    bad.write_bytes(b"RSTX" + p.read_bytes()[4:])
    with pytest.raises(hb.HipBridgeError) as e:
        hb.rstk_read_header(bad)
    assert e.value.code == hb.HB_E_INVALID
    v2 = tmp_path / "v2.bin"
    v2.write_bytes(b"RSTK" + struct.pack("<I", 2) + p.read_bytes()[8:])
    with pytest.raises(hb.HipBridgeError):
        hb.rstk_read_header(v2)
    with pytest.raises(hb.HipBridgeError):
        hb.rstk_read_header(tmp_path / "missing.bin")
    short = tmp_path / "short.bin"
    short.write_bytes(b"RSTK\x01\x00")
    with pytest.raises(hb.HipBridgeError):
        hb.rstk_read_header(short)
