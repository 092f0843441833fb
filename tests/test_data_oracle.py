"""Data path pins (data.rs, bin/train.rs:123-163): compute_bpb known answers,
the position LCG, window placement, and the file readers -- oracle and the
engine's host mirror, no GPU needed."""
import math

import numpy as np
import pytest

import oracle.data as OD
from rustane_amd import engine as E


def test_compute_bpb_known_answers():
    ln2 = math.log(2.0)
    tb = np.array([0, 1, 2, 1, 4], np.int32)
    # every target one byte, every loss ln 2 nats = 1 bit -> 1 bit per byte
    bpb, nats, nbytes = OD.compute_bpb([ln2] * 4, [1, 3, 1, 3], tb)
    assert abs(bpb - 1.0) < 1e-6 and nbytes == 4
    # two-byte targets halve it; special tokens (0 bytes) are skipped entirely
    bpb, nats, nbytes = OD.compute_bpb([ln2, ln2, 5.0], [2, 2, 0], tb)
    assert abs(bpb - 0.5) < 1e-6 and nbytes == 4 and abs(nats - 2 * ln2) < 1e-6
    assert OD.compute_bpb([1.0, 2.0], [0, 0], tb)[0] == 0.0
    # the engine's host mirror computes the same fp32 values
    rng = np.random.default_rng(0)
    losses = rng.random(500).astype(np.float32) * 10
    tg = rng.integers(0, 5, 500)
    a = OD.compute_bpb(losses, tg, tb)
    b = E.compute_bpb(losses, tg, E.TokenBytes(tb))
    assert float(a[0]) == b[0] and float(a[1]) == b[1] and a[2] == b[2]


def test_random_position_lcg():
    assert OD.random_position(3, 2, 1000) == (3 * 7919 + 2 * 104729) % 1000 == 215
    big = 2 ** 63 + 12345  # wrapping u64 arithmetic
    assert OD.random_position(big, 0, 97) == ((big * 7919) % 2 ** 64) % 97
    for s, m in ((0, 0), (17, 3), (123456, 9)):
        assert E.random_position(s, m, 4093) == OD.random_position(s, m, 4093)


def test_window_positions_wrap():
    # n = 100, seq = 10: max_pos = 89; windows at 0, 10, ..., 80, then 90 % 89 = 1
    assert OD.window_positions(100, 10, 11) == [0, 10, 20, 30, 40, 50, 60, 70, 80, 1, 11]


def test_token_files_round_trip(tmp_path):
    toks = np.array([0, 1, 65535, 300, 7], "<u2")
    p = tmp_path / "val.bin"
    toks.tofile(p)
    td = E.TokenData.open(p)
    assert td.len() == 5 and td.token(2) == 65535
    assert td.tokens(1, 3).tolist() == [1, 65535, 300] and td.tokens(1, 3).dtype == np.uint32
    tbp = tmp_path / "token_bytes.bin"
    np.array([3, 0, -1, 7], "<i4").tofile(tbp)
    tb = E.TokenBytes.load(tbp)
    assert [tb.byte_len(i) for i in range(4)] == [3, 0, -1, 7]
