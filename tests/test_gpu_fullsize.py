"""Parity at the full sizes of the benchmark workloads, on the GPU, against the
fp32 oracle on identical seeded weights and tokens.

- 600M shape (1536d / 4096h / 20L, 12 x 128 heads, vocab 32000), seq 512, batch 1 and 8;
- 5B shape (2560d / 6912h / 60L, 20 x 128), seq 512, batch 4;
- 7B shape (4096d / 11008h / 32L, 32 x 128), seq 512 and 2048, batch 1 and 8;
- 7B greedy decode after a 2048-token prefill, batch 1 and 16, teacher-forced.

Weights are N(0, 0.02): the device fills them itself (hb_model_init_synthetic,
stored as fp16) and the oracle regenerates the same values on the host, layer
by layer (tests/_util.SyntheticLayers). Two oracles:

- the weights the device holds: fp32 arithmetic on the fp16-rounded weights.
  Every comparison is made against it, with the bars of the parity contract:
  prefill -- per-position loss within 1e-3 relative, max |dlogit| <= 2e-2;
  greedy decode (teacher-forced) -- max |dlogit| <= 2e-2, top-1 >= 99.5%.
  What remains is the kernels' own arithmetic (fp16 GEMM inputs, fp32
  accumulation, fp16 K/V cache).
- the unrounded fp32 weights, for the first row of each prefill workload.

The kernels round where fp16 MFMA inputs require it (normalised rows, Q/K/V,
attention probabilities and output, SwiGLU gate, final normalised rows), except
in the first layer, which runs on two-term fp16 operands (hi + lo,
hb_model_set_precise_layers, default 1). tests/fp16_emulation_study.py
attributes the distance from fp32 arithmetic per rounding point on the CPU: at
the 7B shape (seq 512, seed 46) rounding inside layer 0 alone carries ~88% of
the logit-error variance (the residual stream is still the small embedding
there, so its relative error is large, and every later layer carries it):

  emulated, vs fp32 on the device's weights   max |dlogit|  max rel dloss  top-1
  fp16 operands everywhere                    3.58e-2       2.09e-3        98.24%
  only layer 0 rounded                        3.49e-2       1.89e-3        98.24%
  layer 0 two-term, the rest fp16             1.32e-2       8.53e-4        99.80%
  layers 0-1 two-term                         9.49e-3       4.92e-4        99.61%

With layer 0 two-term the device meets the contract's bars at every
workload (measured: 600M 3.9e-3 / 2.5e-4; 5B 1.08e-2 / 5.3e-4 / 99.6%; 7B
seq 512 1.43e-2 / 7.7e-4 / 99.4-99.8%, seq 2048 1.34e-2 / 7.4e-4 / 99.71%;
decode 1.21e-2 and 256/257 at batch 1, 1.12e-2 and 256/257 for row 0 of
batch 16; 99.63% top-1 pooled over 11778 positions), so the bars are
applied as stated: logits and per-position
loss on every sequence, greedy top-1 >= 99.5% as a flip rate. Over n compared
positions a rate allows the flips of the 98% quantile of Binomial(n, 0.005)
(flips_allowed: 6 of 512, 17 of 2048), checked per sequence and per test, and
the pooled point estimate over every oracle comparison of the module must
itself reach 99.5% (test_zz_pooled_flip_rate). A bare count bar per sequence
would not test the rate: an implementation exactly at 99.5% flips more than
2 of 512 positions about half the time, and any change of fp32 summation
order anywhere in the model moves which near-tied positions flip (logits move
by ~1e-2 through 32 layers). Two device computations that each meet the
rate (decode against the device's own prefill, batch 16 against batch 1)
are held to twice it. Every comparison is also listed, with its numbers, at
the end of the pytest run (conftest.py's terminal summary).

Decode is compared teacher-forced at each of the benchmark's 256 steps after
the 2048-token prompt, at batch 1 and for row 0 of batch 16. The oracle's
logits for step i are row 2048 + i of one oracle forward over the 2304
tokens (the oracle's decode step at position p is row p of its forward over
tokens 0..p, pinned by test_oracle.py::test_decode_oracle_equals_prefill_rows;
DecodeOracle.step is run for the first steps
on the same cache and checked against those rows), which costs one forward
instead of 256 steps through 26 GB of fp32 weights.

Two device runs of one sequence (batch 8 against batch 1) use different tile
shapes and K splits, so their fp32 sums differ in order; each lies within the
bars of the oracle and their difference is held to twice the bars.

The unrounded-weight comparisons add the weights' own fp16 rounding, which the
workloads define (fp16 weights). The study's --vs-unrounded mode measures
that floor on the 7B sequence above: exact fp32 arithmetic on the fp16
weights is already 3.55e-2 / 2.03e-3 / 98.44% from fp32 arithmetic on the
unrounded weights (the device: 3.75e-2 / 2.09e-3 / 98.05%). Most of it is
again the first layer: keeping the embedding rows and layer 0's weights
unrounded as well would give 1.82e-2 / 8.3e-4 / 98.83% (the other layers'
fp16 weights keep top-1 below 99.5% even with fp32 arithmetic: 1.20e-2 /
7.6e-4 / 99.22%). Those rows are held to BAR_UNROUNDED times the bars, which
checks that the device adds nothing beyond the weights' rounding.
"""
import math
import time

import numpy as np
import pytest

import oracle as O
from rustane_amd import engine as E
from rustane_amd.engine import CompiledKernels, ModelConfig
from tests._util import PARITY, oracle_cfg, synthetic_oracle_weights, tokens_for

pytestmark = pytest.mark.gpu

LOSS_RTOL = 1e-3
LOGIT_ATOL = 2e-2
FLIP_RATE = 0.005          # the contract's greedy top-1 >= 99.5%, as a rate of flips
FLIP_ALPHA = 0.02          # chance that a check fails an implementation exactly at that rate
BAR_DEVICE_PAIR = 2.0      # two device runs of one sequence (see _check_batch)
BAR_UNROUNDED = 2.5        # the weights' own fp16 rounding (module docstring)
UNROUNDED_FLIP_RATE = 0.025
SEED = 1234
STD = 0.02


class _Full:
    """Device model with synthetic weights + the matching lazily generated oracle weights."""

    def __init__(self, cfg, cache_f32=True):
        self.cfg = cfg
        self.k = CompiledKernels.compile(cfg)
        self.k.init_synthetic(SEED, STD)
        self.oc = oracle_cfg(cfg)
        self.ow = synthetic_oracle_weights(cfg, SEED, STD, round16=True)  # what the device holds
        self.ow_f32 = synthetic_oracle_weights(cfg, SEED, STD, cache=cache_f32)

    def forward(self, inp, tgt, B):
        return E.forward_logits(self.cfg, self.k, None, inp, tgt, batch=B)

    def close(self):
        self.k.model.close()
        self.k.ctx.close()
        self.ow = self.ow_f32 = None  # drop the cached host layers


def _tokens(cfg, B, S, seed):
    """B sequences of S+1 uniform tokens; sequence b is stream b of the seed, so the
    first sequence of a batch equals the single sequence drawn with the same seed."""
    return np.stack([tokens_for(cfg, S + 1, seed=seed, stream=b) for b in range(B)])


def flips_allowed(n, rate=FLIP_RATE, alpha=FLIP_ALPHA):
    """Most top-1 flips among n positions consistent with a flip rate of at most
    `rate`: the smallest k with P(Binomial(n, rate) <= k) >= 1 - alpha. A
    top-1 bar is a rate; over n positions the count of flips it allows is a
    quantile, not rate * n (an implementation exactly at 99.5% shows one or
    more flips on 41 positions 19% of the time)."""
    cdf, k = 0.0, 0
    while True:
        cdf += math.comb(n, k) * rate ** k * (1.0 - rate) ** (n - k)
        if cdf >= 1.0 - alpha or k == n:
            return k
        k += 1


def _check_flips(label, same, n, rate=FLIP_RATE):
    flips, allowed = n - same, flips_allowed(n, rate)
    print(f"{label}: top-1 {same}/{n} = {same / n:.4f} ({flips} flips, at most {allowed} "
          f"at a {rate:.1%} flip rate)", flush=True)
    assert flips <= allowed, (label, same, n, allowed)


def _compare(label, V, g_logits, g_losses, r_logits, r_losses, rate=FLIP_RATE,
             bar_scale=1.0, tally=None):
    """Contract bars on one sequence; top-1 agreements are also added to tally
    (a list of (agreeing, positions)) for the test's aggregate check."""
    gl = np.asarray(g_logits).reshape(-1, V)
    rl = np.asarray(r_logits).reshape(-1, V)
    err = float(np.abs(gl - rl).max())
    rel = float((np.abs(np.asarray(g_losses).reshape(-1) - np.asarray(r_losses).reshape(-1))
                 / np.abs(np.asarray(r_losses).reshape(-1))).max())
    same = int((gl.argmax(-1) == rl.argmax(-1)).sum())
    top1 = same / gl.shape[0]
    print(f"{label}: max|dlogit|={err:.3e} max rel dloss={rel:.3e} top1={top1:.4f}", flush=True)
    PARITY.append(dict(label=label, err=err, rel=rel, same=same, n=gl.shape[0],
                       oracle=label.endswith("vs oracle")))
    if label.endswith("vs oracle"):
        _compare.agree.append((same, gl.shape[0]))
    if tally is not None:
        tally.append((same, gl.shape[0]))
    assert err <= LOGIT_ATOL * bar_scale, (label, err)
    assert rel <= LOSS_RTOL * bar_scale, (label, rel)
    _check_flips(label, same, gl.shape[0], rate)


def _check_tally(label, tally, rate=FLIP_RATE):
    _check_flips(label, sum(a for a, _ in tally), sum(b for _, b in tally), rate)


_compare.agree = []  # (agreeing, positions) of every comparison with the oracle


def _oracle_rows(m, ow, tok, rows, label):
    out = {}
    for b in rows:
        t0 = time.time()
        out[b] = O.model_forward(m.oc, ow, tok[b, :-1], tok[b, 1:])
        print(f"{label}: oracle row {b} in {time.time() - t0:.1f} s", flush=True)
    return out


def _check_batch(m, B, S, seed, oracle_rows, label, f32_rows=(0,)):
    """Rows in oracle_rows against the oracle on the device's weights (the
    contract's bars, top-1 per row and over the rows); rows in f32_rows also
    against the unrounded-weight oracle (BAR_UNROUNDED); every other row
    against a batch-1 device forward of the same tokens. Two device runs of one
    sequence differ in fp32 summation order (tile shapes and K splits change
    with the token count), each lies within the bars of the oracle, and the
    difference between them is held to twice the bars (BAR_DEVICE_PAIR)."""
    cfg = m.cfg
    tok = _tokens(cfg, B, S, seed)
    t0 = time.time()
    res = m.forward(tok[:, :-1], tok[:, 1:], B)
    print(f"{label}: device forward B={B} S={S} in {time.time() - t0:.2f} s, loss {res.loss:.5f}",
          flush=True)
    gl = res.logits.reshape(B, S, cfg.vocab)
    gs = res.losses.reshape(B, S)
    refs = _oracle_rows(m, m.ow, tok, oracle_rows, label)
    tally = []
    for b, r in refs.items():
        _compare(f"{label} row {b} vs oracle", cfg.vocab, gl[b], gs[b], r["logits"], r["losses"],
                 tally=tally)
    _check_tally(label, tally)
    for b, r in _oracle_rows(m, m.ow_f32, tok, f32_rows, label + " (unrounded weights)").items():
        _compare(f"{label} row {b} vs unrounded-weight oracle", cfg.vocab, gl[b], gs[b],
                 r["logits"], r["losses"], rate=UNROUNDED_FLIP_RATE, bar_scale=BAR_UNROUNDED)
    for b in range(B):
        if b in refs:
            continue
        one = m.forward(tok[b, :-1], tok[b, 1:], 1)
        _compare(f"{label} row {b} vs batch 1", cfg.vocab, gl[b], gs[b], one.logits, one.losses,
                 bar_scale=BAR_DEVICE_PAIR)
    return res


# ---------------------------------------------------------------------------
# 600M shape
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def m600(gpu):
    m = _Full(ModelConfig.llama_600m())
    yield m
    m.close()


@pytest.mark.timeout(300)
def test_600m_b1_matches_oracle(m600):
    _check_batch(m600, 1, 512, 42, [0], "600M B=1")


@pytest.mark.timeout(300)
def test_600m_b8_matches_oracle(m600):
    _check_batch(m600, 8, 512, 43, range(8), "600M B=8", f32_rows=())


# ---------------------------------------------------------------------------
# 5B shape (60 layers)
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def m5b(gpu, m600):
    m600.close()  # one full-size model on the device at a time
    m = _Full(ModelConfig.llama_5b())
    yield m
    m.close()


@pytest.mark.timeout(400)
def test_5b_b4_matches_oracle(m5b):
    _check_batch(m5b, 4, 512, 44, [0, 3], "5B B=4")


# ---------------------------------------------------------------------------
# 7B shape: prefill at seq 512 and 2048, greedy decode after 2048 positions
# ---------------------------------------------------------------------------
P7 = 2048          # decode prompt = the seq-2048 prefill's tokens
DEC_STEPS = 256    # teacher-forced decode steps checked against the oracle (the benchmark's 256)
DEC_LONG = 256     # free-running greedy steps checked against the device's own prefill
DEC_STEPWISE = 3   # oracle decode steps run one by one, against the oracle forward's rows


@pytest.fixture(scope="module")
def m7b(gpu, m5b):
    m5b.close()
    # seq covers the prompt and the 256 greedy steps (a forward over the whole history)
    m = _Full(ModelConfig.llama_7b(seq=P7 + DEC_LONG), cache_f32=False)  # unrounded weights used once
    yield m
    m.close()


@pytest.fixture(scope="module")
def tok7(m7b):
    """One sequence of P7 + DEC_STEPS + 1 tokens: prompt, targets and teacher-forced inputs."""
    return tokens_for(m7b.cfg, P7 + DEC_STEPS + 1, seed=45)


@pytest.fixture(scope="module")
def orc7(m7b, tok7):
    """Oracle forward over the prompt and the DEC_STEPS teacher-forced tokens
    (prefill_out: logits and losses of all P7 + DEC_STEPS positions), kept as
    a DecodeOracle with every position's K/V cached."""
    orc = O.DecodeOracle(m7b.oc, m7b.ow, ctx_max=P7 + DEC_STEPS)
    t0 = time.time()
    orc.prefill(tok7[:P7 + DEC_STEPS], targets=tok7[1:P7 + DEC_STEPS + 1])
    print(f"7B oracle forward of {P7 + DEC_STEPS} tokens in {time.time() - t0:.1f} s", flush=True)
    return orc


@pytest.fixture(scope="module")
def orc7_steps(m7b, orc7, tok7):
    """Oracle logits of the DEC_STEPS teacher-forced decode steps after the
    prompt: step i (token P7 + i at position P7 + i) is row P7 + i of the
    oracle forward. The first DEC_STEPWISE steps are also run through
    DecodeOracle.step, rewound to position P7 on the same K/V cache, and must
    give those rows (to fp32 summation order)."""
    V = m7b.cfg.vocab
    rows = orc7.prefill_out["logits"].reshape(P7 + DEC_STEPS, V)[P7:]
    orc7.pos = P7
    t0 = time.time()
    for i in range(DEC_STEPWISE):
        d = float(np.abs(orc7.step(int(tok7[P7 + i])) - rows[i]).max())
        print(f"7B oracle decode step {i} vs oracle forward row {P7 + i}: max|dlogit| {d:.2e}", flush=True)
        assert d <= 1e-3, (i, d)
    print(f"7B oracle: {DEC_STEPWISE} decode steps in {time.time() - t0:.1f} s", flush=True)
    return [rows[i] for i in range(DEC_STEPS)]


def _oracle_prefix(orc7, V):
    """The oracle forward restricted to the first P7 positions (causal: rows < P7
    of the longer forward are the P7-token forward's rows)."""
    out = orc7.prefill_out
    losses = np.asarray(out["losses"]).reshape(-1)[:P7]
    return out["logits"].reshape(-1, V)[:P7], losses, float(np.float64(losses).mean())


@pytest.mark.timeout(400)
def test_7b_s512_b1_matches_oracle(m7b):
    _check_batch(m7b, 1, 512, 46, [0], "7B S=512 B=1")


@pytest.mark.timeout(300)
def test_7b_s512_b8_matches_oracle(m7b):
    _check_batch(m7b, 8, 512, 47, [0, 7], "7B S=512 B=8", f32_rows=())


@pytest.mark.timeout(600)
def test_7b_s2048_b1_matches_oracle(m7b, tok7, orc7):
    cfg = m7b.cfg
    res = m7b.forward(tok7[:P7], tok7[1:P7 + 1], 1)
    r_logits, r_losses, r_loss = _oracle_prefix(orc7, cfg.vocab)
    tally = []
    _compare("7B S=2048 B=1 vs oracle", cfg.vocab, res.logits, res.losses, r_logits, r_losses, tally=tally)
    _check_tally("7B S=2048 B=1", tally)
    assert abs(res.loss - r_loss) <= LOSS_RTOL * r_loss


@pytest.mark.timeout(300)
def test_7b_s2048_b8_matches_oracle(m7b, tok7, orc7):
    """Row 0 of the batch is the oracle's sequence; rows 1 and 7 are checked
    against batch-1 device forwards of the same tokens."""
    cfg, B = m7b.cfg, 8
    tok = np.stack([tok7[:P7 + 1]] + [tokens_for(cfg, P7 + 1, seed=48, stream=b) for b in range(1, B)])
    res = m7b.forward(tok[:, :-1], tok[:, 1:], B)
    gl = res.logits.reshape(B, P7, cfg.vocab)
    gs = res.losses.reshape(B, P7)
    r_logits, r_losses, _ = _oracle_prefix(orc7, cfg.vocab)
    tally = []
    _compare("7B S=2048 B=8 row 0 vs oracle", cfg.vocab, gl[0], gs[0], r_logits, r_losses, tally=tally)
    _check_tally("7B S=2048 B=8", tally)
    for b in (1, B - 1):
        one = m7b.forward(tok[b, :-1], tok[b, 1:], 1)
        _compare(f"7B S=2048 B=8 row {b} vs batch 1", cfg.vocab, gl[b], gs[b], one.logits, one.losses,
                 bar_scale=BAR_DEVICE_PAIR)


@pytest.mark.timeout(400)
def test_7b_decode_b1_teacher_forced_matches_oracle(m7b, tok7, orc7, orc7_steps):
    cfg = m7b.cfg
    dec = E.Decoder(m7b.k, batch=1, ctx_max=P7 + DEC_STEPS)
    try:
        gl, gn = dec.prefill(tok7[:P7])
        rl = _oracle_prefix(orc7, cfg.vocab)[0][-1]
        errs, agree = [float(np.abs(gl[0] - rl).max())], [int(gn[0]) == int(rl.argmax())]
        for i in range(DEC_STEPS):
            gl, gn = dec.step([tok7[P7 + i]])
            rl = orc7_steps[i]
            errs.append(float(np.abs(gl[0] - rl).max()))
            agree.append(int(gn[0]) == int(rl.argmax()))
            assert int(gn[0]) == int(gl[0].argmax())
        print(f"7B decode B=1 after {P7}: max|dlogit|={max(errs):.3e}", flush=True)
        PARITY.append(dict(label=f"7B decode B=1, {DEC_STEPS} teacher-forced steps vs oracle", err=max(errs),
                           rel=None, same=int(sum(agree)), n=len(agree), oracle=True))
        assert max(errs) <= LOGIT_ATOL
        _compare.agree.append((int(sum(agree)), len(agree)))
        _check_flips(f"7B decode B=1 after {P7} vs oracle", int(sum(agree)), len(agree))
        assert dec.length() == P7 + DEC_STEPS
    finally:
        dec.kv.close()


@pytest.mark.timeout(400)
def test_7b_decode_b16_rows_match_oracle_and_batch_one(m7b, tok7, orc7, orc7_steps):
    """Batch 16: row 0 carries the oracle's sequence (teacher-forced: its logits
    and its greedy token compared with the oracle at every one of the 256
    steps); row 15 is compared with a batch-1 decoder fed the same tokens,
    greedy token included."""
    cfg, B, n = m7b.cfg, 16, DEC_STEPS
    others = [tokens_for(cfg, P7 + n, seed=49, stream=b) for b in range(1, B)]
    tok = np.stack([tok7[:P7 + n]] + others)
    db = E.Decoder(m7b.k, batch=B, ctx_max=P7 + n)
    d1 = E.Decoder(m7b.k, batch=1, ctx_max=P7 + n)
    try:
        lb, nb = db.prefill(tok[:, :P7])
        l1, _ = d1.prefill(tok[B - 1, :P7])
        rl = _oracle_prefix(orc7, cfg.vocab)[0][-1]
        errs = [float(np.abs(lb[0] - rl).max())]
        agree0 = [int(nb[0]) == int(rl.argmax())]
        cross = [float(np.abs(lb[B - 1] - l1[0]).max())]
        same1 = int(int(lb[B - 1].argmax()) == int(l1[0].argmax()))
        for i in range(n):
            lb, nb = db.step(tok[:, P7 + i])
            l1, _ = d1.step([tok[B - 1, P7 + i]])
            errs.append(float(np.abs(lb[0] - orc7_steps[i]).max()))
            agree0.append(int(nb[0]) == int(orc7_steps[i].argmax()))
            cross.append(float(np.abs(lb[B - 1] - l1[0]).max()))
            assert int(nb[0]) == int(lb[0].argmax())
            same1 += int(int(nb[B - 1]) == int(l1[0].argmax()))
        print(f"7B decode B=16: row 0 vs oracle max|dlogit|={max(errs):.3e}; row 15 vs batch 1 "
              f"{max(cross):.3e}", flush=True)
        PARITY.append(dict(label=f"7B decode B=16 row 0, {n} teacher-forced steps vs oracle", err=max(errs),
                           rel=None, same=int(sum(agree0)), n=len(agree0), oracle=True))
        PARITY.append(dict(label="7B decode B=16 row 15 vs batch 1", err=max(cross), rel=None, same=same1,
                           n=n + 1, oracle=False))
        assert max(errs) <= LOGIT_ATOL
        assert max(cross) <= LOGIT_ATOL
        _compare.agree.append((int(sum(agree0)), len(agree0)))
        _check_flips("7B decode B=16 row 0 vs oracle", int(sum(agree0)), len(agree0))
        _check_flips("7B decode B=16 row 15 vs batch 1", same1, n + 1, rate=2 * FLIP_RATE)
    finally:
        db.kv.close()
        d1.kv.close()


def _greedy_against_prefill(m7b, B, rows, seed):
    """The benchmark's decode workload: B sequences, a 2048-token seeded
    prompt, then 256 free-running greedy steps, each feeding back its own
    argmax (the step's logits are kept). A forward over each checked row's
    whole history (prompt + the fed-back tokens) must give the same logits at
    every decoded position, within the contract's 2e-2, and the same greedy
    token at >= 99% of them: decode (GEMV, one position) and prefill (GEMM,
    all positions) are two device computations in different summation orders,
    each at its own distance from the oracle (both checked against it above),
    so near-tied logits can flip between them (measured: 254/256 at batch 1,
    511/512 at batch 16). The captured greedy graph must produce the same
    tokens as the step-by-step decode."""
    cfg = m7b.cfg
    prompt = np.stack([tokens_for(cfg, P7, seed=seed, stream=b) for b in range(B)])
    dec = E.Decoder(m7b.k, batch=B, ctx_max=P7 + DEC_LONG)
    dg = E.Decoder(m7b.k, batch=B, ctx_max=P7 + DEC_LONG)
    try:
        t0 = time.time()
        gl, nxt = dec.prefill(prompt)
        hist, logits = [nxt.copy()], {b: [gl[b].copy()] for b in rows}
        for i in range(DEC_LONG - 1):
            gl, nxt = dec.step(hist[-1])
            hist.append(nxt.copy())
            for b in rows:
                logits[b].append(gl[b].copy())
        hist = np.stack(hist, axis=1)  # [B, DEC_LONG]: tokens at positions P7 .. P7+DEC_LONG-1
        print(f"7B decode B={B}: prefill + {DEC_LONG - 1} steps in {time.time() - t0:.1f} s", flush=True)
        _, n0 = dg.prefill(prompt)
        graph_tokens = dg.greedy(n0, DEC_LONG - 1)  # [steps, B]
        np.testing.assert_array_equal(graph_tokens.T, hist[:, 1:])
    finally:
        dec.kv.close()
        dg.kv.close()
    tally = []
    for b in rows:
        seq = np.concatenate([prompt[b], hist[b, :-1]])  # positions 0 .. P7+DEC_LONG-2
        full = m7b.forward(seq, None, 1).logits.reshape(-1, cfg.vocab)
        rows_ref = full[P7 - 1:]  # logits at positions P7-1 .. P7+DEC_LONG-2
        got = np.stack(logits[b])
        err = float(np.abs(got - rows_ref).max())
        same = int((got.argmax(-1) == rows_ref.argmax(-1)).sum())
        tally.append((same, got.shape[0]))
        print(f"7B decode B={B} row {b}: {got.shape[0]} decoded positions vs device prefill rows: "
              f"max|dlogit|={err:.3e} top1 {same}/{got.shape[0]}", flush=True)
        PARITY.append(dict(label=f"7B greedy B={B} row {b}, {got.shape[0]} steps vs device prefill rows",
                           err=err, rel=None, same=same, n=got.shape[0], oracle=False))
        assert err <= LOGIT_ATOL
    _check_tally(f"7B decode B={B} vs prefill rows", tally, rate=2 * FLIP_RATE)


@pytest.mark.timeout(600)
def test_7b_greedy_256_steps_b1_equal_prefill_rows(m7b):
    _greedy_against_prefill(m7b, 1, [0], seed=50)


@pytest.mark.timeout(600)
def test_7b_greedy_256_steps_b16_equal_prefill_rows(m7b):
    _greedy_against_prefill(m7b, 16, [0, 15], seed=51)


def test_zz_pooled_flip_rate():
    """Every comparison with the oracle that ran in this module, pooled: the
    contract's 99.5% top-1 as a rate over all compared positions."""
    if not _compare.agree:
        pytest.skip("no oracle comparison ran")
    same, n = sum(a for a, _ in _compare.agree), sum(c for _, c in _compare.agree)
    _check_flips("all oracle comparisons", same, n)
    assert same / n >= 1.0 - FLIP_RATE, (same, n)  # the contract's 99.5%, as a point estimate
