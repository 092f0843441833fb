"""Data path and validation of rustane (TEST INFRASTRUCTURE ONLY):
crates/engine/src/data.rs and the validate loop of bin/train.rs:123-163,
restated on top of the forward oracle. Pins: tests/test_data_oracle.py."""
from __future__ import annotations

import math

import numpy as np

from .forward import model_forward

F32 = np.float32


def compute_bpb(losses, targets, token_bytes):
    """data.rs:61-83: fp32 sum of the losses of targets with a positive byte
    length, integer sum of those lengths; bpb = nats / (ln 2 * bytes), 0 if no
    bytes. Returns (bpb, total_nats, total_bytes)."""
    tb = np.asarray(token_bytes)
    nats = F32(0.0)
    nbytes = 0
    for loss, tok in zip(np.asarray(losses, F32), np.asarray(targets)):
        bl = int(tb[int(tok)])
        if bl > 0:
            nats = F32(nats + loss)
            nbytes += bl
    if nbytes == 0:
        return F32(0.0), nats, 0
    return F32(nats / F32(F32(math.log(2.0)) * F32(nbytes))), nats, nbytes


def random_position(step: int, micro: int, max_pos: int) -> int:
    """data.rs:86-90: (step*7919 + micro*104729) % max_pos in wrapping u64."""
    m = (1 << 64) - 1
    return (((step * 7919) & m) + ((micro * 104729) & m) & m) % max_pos


def window_positions(n_tokens: int, seq: int, steps: int):
    """bin/train.rs:133-137: window vs starts at (vs * seq) % (n - seq - 1)."""
    max_pos = n_tokens - seq - 1
    return [(vs * seq) % max_pos for vs in range(steps)]


def validate(cfg, w, tokens, token_bytes, steps: int, softcap: float = 0.0):
    """bin/train.rs:123-163 with forward_losses = the oracle's forward:
    returns (avg_loss, bpb, total_nats, total_bytes)."""
    toks = np.asarray(tokens)
    seq = cfg.seq
    total_loss = F32(0.0)
    losses_all, targets_all = [], []
    for pos in window_positions(toks.size, seq, steps):
        inp = toks[pos:pos + seq].astype(np.int64)
        tgt = toks[pos + 1:pos + 1 + seq].astype(np.int64)
        out = model_forward(cfg, w, inp, tgt, softcap, want_logits=False)
        total_loss = F32(total_loss + out["losses"].sum(dtype=F32))
        losses_all.append(out["losses"])
        targets_all.append(tgt)
    avg = F32(total_loss / F32(steps * seq))
    if token_bytes is None:
        return avg, F32(0.0), F32(0.0), 0
    bpb, nats, nbytes = compute_bpb(np.concatenate(losses_all), np.concatenate(targets_all), token_bytes)
    return avg, bpb, nats, nbytes
