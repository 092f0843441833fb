"""Training forward + backward on the GPU (hb_forward_backward) against the
backward oracle (oracle/backward.py, pinned by torch float64 autograd in
tests/test_backward_oracle.py) on the same fp16-rounded weights.

The device runs every product on fp16 MFMA inputs with fp32 accumulation (the
activations, dlogits, dQKV, dH13 and attention probabilities are rounded to
fp16 where they enter a GEMM), the oracle in fp32 throughout, so gradients
agree to the fp16 rounding of those operands, not bit for bit. The bars below
are per tensor:
    max |dev - ref| <= GRAD_MAX_REL * max |ref|
    ||dev - ref||_2 <= GRAD_L2_REL  * ||ref||_2
and the loss within LOSS_RTOL. Accumulation (two calls add exactly twice one
call) and run-to-run determinism are checked bit for bit.
"""
import numpy as np
import pytest

import oracle as O
import oracle.backward as OB
from rustane_amd import engine as E
from rustane_amd import hip_bridge as hb
from rustane_amd.engine import CompiledKernels, ModelConfig, ModelWeights
from tests._util import F32, f16_round, oracle_cfg, tiny_config, tokens_for

pytestmark = pytest.mark.gpu

# measured worst cases: max-rel 1.34e-3, l2-rel 1.24e-3 (tiny softcap, 48M)
GRAD_MAX_REL = 5e-3
GRAD_L2_REL = 5e-3
LOSS_RTOL = 1e-3


def _rounded_oracle_weights(w: ModelWeights):
    ow = O.ModelW.of(w)
    return O.ModelW(embed=f16_round(ow.embed), gamma_final=ow.gamma_final,
                    layers=[O.LayerW(**{k: (f16_round(getattr(l, k)) if k.startswith("w") else getattr(l, k))
                                        for k in O.LayerW.__dataclass_fields__}) for l in ow.layers])


def _oracle(cfg, ow, tok, tgt, B, S, softcap, loss_scale):
    """Sum over the B sequences of the oracle's per-sequence gradients."""
    ocfg = oracle_cfg(cfg)
    tot, losses, acc = None, [], None
    for b in range(B):
        loss, g = OB.model_forward_backward(ocfg, ow, tok[b * S:(b + 1) * S], tgt[b * S:(b + 1) * S],
                                            softcap, loss_scale)
        losses.append(loss)
        if acc is None:
            acc = g
        else:
            acc["embed"] = acc["embed"] + g["embed"]
            acc["gamma_final"] = acc["gamma_final"] + g["gamma_final"]
            for a, c in zip(acc["layers"], g["layers"]):
                for k in OB.LAYER_TENSORS:
                    a[k] = a[k] + c[k]
    return float(np.mean(losses)), acc


def _device_grads(opt, nlayers):
    e, gf = opt.download_embed(hb.Optimizer.GRADS)
    return {"embed": e, "gamma_final": gf,
            "layers": [opt.download_layer(l, hb.Optimizer.GRADS) for l in range(nlayers)]}


def _pairs(dev, ref):
    out = [("embed", dev["embed"], ref["embed"]), ("gamma_final", dev["gamma_final"], ref["gamma_final"])]
    for l, (a, b) in enumerate(zip(dev["layers"], ref["layers"])):
        out += [(f"{l}.{k}", a[k], b[k]) for k in OB.LAYER_TENSORS]
    return out


def _compare(dev, ref, label):
    worst_max, worst_l2 = 0.0, 0.0
    fails = []
    for name, a, b in _pairs(dev, ref):
        a = np.asarray(a, np.float64).reshape(-1)
        b = np.asarray(b, np.float64).reshape(-1)
        emax = np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)
        el2 = np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)
        worst_max, worst_l2 = max(worst_max, emax), max(worst_l2, el2)
        if emax > GRAD_MAX_REL or el2 > GRAD_L2_REL:
            fails.append((name, emax, el2))
    print(f"{label}: worst max-rel {worst_max:.3e}, worst l2-rel {worst_l2:.3e}", flush=True)
    assert not fails, fails


def _run_case(cfg, B, S, seed, softcap=0.0, loss_scale=256.0, std=0.02):
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=seed, std=std)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        k.set_softcap(softcap)
        tok = tokens_for(cfg, B * S + 1, seed=seed + 100)
        tokens, targets = tok[:-1], tok[1:]
        print(f"case dim={cfg.dim} L={cfg.nlayers} H={cfg.heads}/{cfg.kv_heads} B={B} S={S} "
              f"softcap={softcap}", flush=True)
        st.opt.zero_grads()
        mean, losses = st.opt.forward_backward(tokens, targets, B, S, loss_scale, want_losses=True)
        dev = _device_grads(st.opt, cfg.nlayers)
        ref_loss, ref = _oracle(cfg, _rounded_oracle_weights(w), tokens, targets, B, S, softcap,
                                loss_scale)
        print(f"loss device {mean:.6f} oracle {ref_loss:.6f}", flush=True)
        assert abs(mean - ref_loss) <= LOSS_RTOL * ref_loss
        assert abs(float(np.mean(losses)) - mean) <= 1e-5 * mean
        _compare(dev, ref, f"B={B} S={S}")
        return k, st, tokens, targets, dev
    except BaseException:
        st.close()
        raise


def test_tiny_mha_full_sequence():
    cfg = tiny_config()
    _, st, *_ = _run_case(cfg, 1, cfg.seq, seed=11)
    st.close()


def test_long_sequence_attention_kernels_hd128():
    """Enough (query block, head, sequence) groups -- 16 sequences of 500 at 8
    heads of 128 -- that the attention kernels take the variants the 7B shape
    runs at one sequence of 2048: the forward and the dQ kernel with 8 query
    blocks per workgroup, dK/dV with 4 key blocks; S = 500 keeps the padding
    rows."""
    cfg = tiny_config(dim=1024, hidden=512, heads=8, kv_heads=8, hd=128, nlayers=1, seq=512, vocab=512)
    _, st, *_ = _run_case(cfg, 16, 500, seed=21)
    st.close()


def test_long_sequence_attention_kernels_hd64_gqa():
    """The same at hd = 64 with GQA 16/8: dQ with 4 query blocks per
    workgroup (8 is for hd = 128), dK/dV summing two query heads per group."""
    cfg = tiny_config(dim=1024, hidden=512, heads=16, kv_heads=8, hd=64, nlayers=1, seq=512, vocab=512)
    _, st, *_ = _run_case(cfg, 16, 500, seed=22)
    st.close()


def test_tiny_gqa_two_sequences_ragged_length():
    """GQA (dK/dV summed over each group's query heads) and S = 33, not a
    multiple of 64, so every padding row and column is exercised."""
    cfg = tiny_config(heads=4, kv_heads=2)
    _, st, *_ = _run_case(cfg, 2, 33, seed=12)
    st.close()


def test_head_dim_128_gqa():
    """hd = 128, the 7B/600M head size (the other cases use 64), with GQA."""
    cfg = tiny_config(dim=256, hidden=512, heads=4, kv_heads=2, hd=128)
    _, st, *_ = _run_case(cfg, 2, 37, seed=26)
    st.close()


def test_tiny_softcap():
    """Logits of about one softcap in size (|z|/c ~ 1), where tanh bends but
    does not saturate. Deep in saturation the factor 1 - t^2 turns the fp16
    GEMMs' relative logit error e into a relative gradient error of about
    2 e |z| / c (|z|/c ~ 10 with std-0.3 weights gives ~2%), a property of the
    fp16 forward, not of the backward."""
    cfg = tiny_config()
    _, st, *_ = _run_case(cfg, 1, cfg.seq, seed=13, softcap=0.5, std=0.05)
    st.close()


def test_48m_shape():
    cfg = ModelConfig.llama_48m()
    _, st, *_ = _run_case(cfg, 1, 128, seed=14)
    st.close()


def test_many_sequences_long_token_dimension():
    """26 sequences of 40: 1040 tokens, so the weight-gradient products have
    K = 1088 > 1024 and take the 256x256 tiles (with the gradient-norm sums)
    instead of the short-K 128x128 ones."""
    cfg = tiny_config()
    k, st, *_ = _run_case(cfg, 26, cfg.seq, seed=32)
    try:
        fused = st.opt.grad_norm()
        dev = _device_grads(st.opt, cfg.nlayers)
        ref = np.sqrt(sum(float(np.sum(np.asarray(a, np.float64) ** 2)) for _, a, _ in _pairs(dev, dev)))
        print(f"B=26: fused norm {fused:.7e} float64 {ref:.7e}", flush=True)
        assert abs(fused - ref) <= 1e-6 * ref
    finally:
        st.close()


def test_bars_catch_planted_oracle_mistakes():
    """The same device gradients against an oracle with a plausible mistake
    planted (on the CPU): the softmax-backward row sum dropped, the forward
    RoPE rotation used for its inverse, the residual alpha left out. Each must
    break the bars above."""
    cfg = tiny_config()
    k, st, tokens, targets, dev = _run_case(cfg, 1, cfg.seq, seed=18)
    st.close()
    ow = _rounded_oracle_weights(ModelWeights.synthetic(cfg, seed=18, std=0.02))
    orig_sdpa, orig_rope, orig_layer = OB.sdpa_backward, OB.rope_backward_cf, OB.layer_backward

    def no_row_sum(cfg_, q, kk, v, da, seq):
        H, hd = cfg_.heads, cfg_.hd
        scale = F32(1.0) / np.sqrt(F32(hd))
        qh, kh, vh, dh = (np.asarray(a, F32).reshape(H, hd, seq).transpose(0, 2, 1) for a in (q, kk, v, da))
        sc = (qh @ kh.transpose(0, 2, 1)) * scale + O.causal_mask(seq)[None]
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        ds = p * (dh @ vh.transpose(0, 2, 1)) * scale
        cf = lambda t: np.ascontiguousarray(t.transpose(0, 2, 1)).reshape(H * hd, seq).astype(F32)
        return cf(ds @ kh), cf(ds.transpose(0, 2, 1) @ qh), cf(p.transpose(0, 2, 1) @ dh)

    def forward_rotation(dx, heads, hd, seq, theta=10000.0):
        return O.rope_apply_cf(dx, heads, hd, seq, *O.rope_table(seq, hd, theta))

    def no_alpha(cfg_, lw, taps, x_in, dy, seq):
        return orig_layer(O.Config(**{**cfg_.__dict__, "residual_alpha": 1.0}), lw, taps, x_in, dy, seq)

    for name, fn in (("sdpa_backward", no_row_sum), ("rope_backward_cf", forward_rotation),
                     ("layer_backward", no_alpha)):
        setattr(OB, name, fn)
        try:
            _, ref = _oracle(cfg, ow, tokens, targets, 1, cfg.seq, 0.0, 256.0)
            with pytest.raises(AssertionError):
                _compare(dev, ref, f"planted {name}")
        finally:
            OB.sdpa_backward, OB.rope_backward_cf, OB.layer_backward = orig_sdpa, orig_rope, orig_layer


def test_accumulation_and_determinism():
    cfg = tiny_config(heads=4, kv_heads=1)
    k, st, tokens, targets, one = _run_case(cfg, 2, cfg.seq, seed=15)
    try:
        st.opt.forward_backward(tokens, targets, 2, cfg.seq, 256.0)
        two = _device_grads(st.opt, cfg.nlayers)
        for name, a, b in _pairs(two, one):
            if name == "embed":
                # two additions per call (the dE product, then the token
                # scatter-add): ((G + S) + G) + S is 2 (G + S) to fp32 rounding
                np.testing.assert_allclose(a, np.asarray(b, F32) * 2, rtol=2e-6, atol=1e-7, err_msg=name)
            else:
                np.testing.assert_array_equal(a, np.asarray(b, F32) * 2, err_msg=name)
        st.opt.zero_grads()
        st.opt.forward_backward(tokens, targets, 2, cfg.seq, 256.0)
        again = _device_grads(st.opt, cfg.nlayers)
        for name, a, b in _pairs(again, one):
            np.testing.assert_array_equal(a, b, err_msg=name)
    finally:
        st.close()


def test_train_steps_lower_the_loss():
    """hb_forward_backward + hb_opt_step as train_step (full_model.rs:661-714)
    repeated on one batch: the loss must fall."""
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=16, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(max_lr=3e-3, warmup_steps=1, total_steps=100), weights=w)
    try:
        tok = tokens_for(cfg, cfg.seq + 1, seed=99)
        losses = []
        for step in range(8):
            st.opt.zero_grads()
            losses.append(st.opt.forward_backward(tok[:-1], tok[1:], 1, cfg.seq, 256.0))
            st.opt.step(step, want_norm=False)
        print("losses", [f"{x:.4f}" for x in losses], flush=True)
        assert losses[-1] < losses[0] - 0.05
        # the weights the forward reads changed with the steps
        after = E.forward_logits(cfg, k, None, tok[:-1], tok[1:])
        assert abs(float(np.mean(after.losses)) - losses[-1]) < 0.5
    finally:
        st.close()


def test_engine_train_step_accumulates_the_microbatches():
    """engine.train_step (full_model.rs:661-714): accum_steps windows at the
    LCG positions of full_model.rs:682, their gradients summed in the arena
    (compared with the oracle's sum over the same windows), the mean loss
    returned, then the update."""
    import oracle.data as OD
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=19, std=0.02)
    tc = E.TrainConfig(accum_steps=3, warmup_steps=2, total_steps=50)
    st = E.ModelOptState(k, tc, weights=w)
    try:
        data = tokens_for(cfg, 600, seed=7).astype(np.uint16)
        step = 5
        loss = E.train_step(cfg, k, st, data, step, tc)
        dev = _device_grads(st.opt, cfg.nlayers)
        ow = _rounded_oracle_weights(w)
        max_pos = len(data) - cfg.seq - 1
        toks, tgts = [], []
        for micro in range(tc.accum_steps):
            pos = OD.random_position(step, micro, max_pos)
            toks.append(data[pos:pos + cfg.seq])
            tgts.append(data[pos + 1:pos + cfg.seq + 1])
        ref_loss, ref = _oracle(cfg, ow, np.concatenate(toks), np.concatenate(tgts), tc.accum_steps,
                                cfg.seq, 0.0, tc.loss_scale)
        print(f"train_step loss {loss:.6f} oracle {ref_loss:.6f}", flush=True)
        assert abs(loss - ref_loss) <= LOSS_RTOL * ref_loss
        _compare(dev, ref, "train_step arena")
        # the update moved the master weights
        assert np.abs(st.opt.download_layer(0, hb.Optimizer.WEIGHTS)["w2"] - w.layers[0].w2).max() > 0
        with pytest.raises(ValueError):
            E.train_step(cfg, k, st, data, step, E.TrainConfig())
    finally:
        st.close()


def test_optimizer_update_keeps_transposed_weights_current():
    """Once a model trains, hb_opt updates its matrices with the tiled AdamW
    kernel that also writes the transposed fp16 copies the backward reads:
    weights and moments stay bit-exact with the oracle, and a backward after
    the update equals, bit for bit, one on a fresh model uploaded with the
    updated master weights (whose transposes are built from scratch)."""
    import oracle.optimizer as OP
    cfg = tiny_config(heads=4, kv_heads=2)
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=20, std=0.02)
    tc = E.TrainConfig()
    st = E.ModelOptState(k, tc, weights=w)
    k2 = st2 = None
    try:
        tok = tokens_for(cfg, 2 * cfg.seq + 1, seed=21)
        st.opt.zero_grads()
        st.opt.forward_backward(tok[:-1], tok[1:], 2, cfg.seq, 256.0)
        g = _device_grads(st.opt, cfg.nlayers)
        ref = {"embed": np.array(w.embed, F32), "gamma_final": np.array(w.gamma_final, F32),
               "layers": [{kk: np.array(getattr(lw, kk), F32) for kk in OP.LAYER_TENSORS} for lw in w.layers]}
        mom = {"m": OP.zeros_like_state(ref), "v": OP.zeros_like_state(ref)}
        for t in (1, 2):
            OP.update_weights(ref, g, mom, t, F32(3e-3), tc, F32(1.0 / 256.0))
            st.opt.update_weights(t, 3e-3, 1.0 / 256.0)
        for which, want in ((hb.Optimizer.WEIGHTS, ref), (hb.Optimizer.M, mom["m"]), (hb.Optimizer.V, mom["v"])):
            e, gf = st.opt.download_embed(which)
            np.testing.assert_array_equal(e, want["embed"], err_msg=f"embed {which}")
            for l in range(cfg.nlayers):
                got = st.opt.download_layer(l, which)
                for kk in OP.LAYER_TENSORS:
                    np.testing.assert_array_equal(got[kk], want["layers"][l][kk], err_msg=f"{l}.{kk} {which}")
        st.opt.zero_grads()
        st.opt.forward_backward(tok[:-1], tok[1:], 2, cfg.seq, 256.0)
        after = _device_grads(st.opt, cfg.nlayers)
        # a fresh model with the updated master weights
        e, gf = st.opt.download_embed(hb.Optimizer.WEIGHTS)
        lws = [st.opt.download_layer(l, hb.Optimizer.WEIGHTS) for l in range(cfg.nlayers)]
        w2 = ModelWeights(embed=e, gamma_final=gf, layers=[E.LayerWeights(**lw) for lw in lws])
        k2 = CompiledKernels.compile(cfg)
        st2 = E.ModelOptState(k2, tc, weights=w2)
        st2.opt.zero_grads()
        st2.opt.forward_backward(tok[:-1], tok[1:], 2, cfg.seq, 256.0)
        fresh = _device_grads(st2.opt, cfg.nlayers)
        for name, a, b in _pairs(after, fresh):
            np.testing.assert_array_equal(a, b, err_msg=name)
    finally:
        st.close()
        if st2 is not None:
            st2.close()


def test_shape_changes_leave_no_stale_padding():
    """One model trained at (1, 40), then (2, 33), (3, 21) and (3, 1) -- one
    token per sequence -- then (1, 40) again: the training buffers are reused
    or regrown and re-zeroed on every shape change, so the last call
    reproduces the first bit for bit, and the other shapes agree with the
    oracle."""
    cfg = tiny_config(heads=4, kv_heads=2)
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=22, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        tok = tokens_for(cfg, 3 * cfg.seq + 1, seed=23)
        ow = _rounded_oracle_weights(w)
        runs = {}
        for B, S in ((1, cfg.seq), (2, 33), (3, 21), (3, 1), (1, cfg.seq)):
            st.opt.zero_grads()
            n = B * S
            st.opt.forward_backward(tok[:n], tok[1:n + 1], B, S, 256.0)
            dev = _device_grads(st.opt, cfg.nlayers)
            if (B, S) in runs:
                for name, a, b in _pairs(dev, runs[(B, S)]):
                    np.testing.assert_array_equal(a, b, err_msg=name)
            else:
                runs[(B, S)] = dev
                _, ref = _oracle(cfg, ow, tok[:n], tok[1:n + 1], B, S, 0.0, 256.0)
                _compare(dev, ref, f"B={B} S={S}")
    finally:
        st.close()


def test_writes_through_the_raw_arena_pointer_are_kept():
    """After hb_opt_grad_arena hands out the pointer, a zeroed arena may be
    written by the caller, so the backward must add to it, not overwrite."""
    import torch
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=24, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        tok = tokens_for(cfg, cfg.seq + 1, seed=25)
        st.opt.zero_grads()
        st.opt.forward_backward(tok[:-1], tok[1:], 1, cfg.seq, 256.0)
        base = _device_grads(st.opt, cfg.nlayers)
        ptr, n = st.opt.grad_arena()
        st.opt.zero_grads()

        class _Arr:
            __cuda_array_interface__ = {"shape": (n,), "typestr": "<f4", "data": (ptr, False), "version": 3}
        torch.as_tensor(_Arr(), device="cuda").fill_(0.5)
        torch.cuda.synchronize()
        st.opt.forward_backward(tok[:-1], tok[1:], 1, cfg.seq, 256.0)
        got = _device_grads(st.opt, cfg.nlayers)
        for name, a, b in _pairs(got, base):
            if name == "embed":
                np.testing.assert_allclose(a, np.asarray(b, F32) + F32(0.5), rtol=1e-6, atol=1e-6, err_msg=name)
            else:
                np.testing.assert_array_equal(a, np.asarray(b, F32) + F32(0.5), err_msg=name)
    finally:
        st.close()


def test_lazy_zero_grads_reads_as_zero():
    """hb_opt_zero_grads defers the clearing to the first consumer: reads,
    partial uploads and norms see zeros, and a training backward overwrites
    every element."""
    import oracle.optimizer as OP
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=27, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        rng = np.random.default_rng(28)
        noise = {kk: rng.standard_normal(v.size).astype(F32) for kk, v in st.opt.download_layer(0, 3).items()}
        for l in range(cfg.nlayers):
            st.opt.upload_grads_layer(l, noise)
        st.opt.zero_grads()
        assert st.opt.grad_norm() == 0.0
        st.opt.upload_grads_layer(1, noise)
        st.opt.zero_grads()
        st.opt.upload_grads_layer(0, noise)  # partial write onto a lazily zeroed arena
        ref = np.sqrt(sum(float(np.sum(v.astype(np.float64) ** 2)) for v in noise.values()))
        assert abs(st.opt.grad_norm() - ref) <= 1e-6 * ref
        for kk, v in st.opt.download_layer(1, 3).items():
            assert not v.any(), kk
        # zero, then a backward: equal to the backward on a freshly created optimizer
        tok = tokens_for(cfg, cfg.seq + 1, seed=29)
        st.opt.zero_grads()
        st.opt.forward_backward(tok[:-1], tok[1:], 1, cfg.seq, 256.0)
        got = _device_grads(st.opt, cfg.nlayers)
        st2 = E.ModelOptState(k, E.TrainConfig(), weights=w)
        try:
            st2.opt.forward_backward(tok[:-1], tok[1:], 1, cfg.seq, 256.0)
            for name, a, b in _pairs(got, _device_grads(st2.opt, cfg.nlayers)):
                np.testing.assert_array_equal(a, b, err_msg=name)
        finally:
            st2.close()
    finally:
        st.close()


def test_gradient_norm_from_backward_partials():
    """After a training backward the norm is assembled from sums of squares
    taken while the gradients were written (per weight-gradient tile, per
    gamma block, plus the embedding after its scatter-add) instead of a
    second pass over the arena: equal to the float64 norm of the downloaded
    gradients and to the full pass, after a stored and an accumulated call."""
    cfg = tiny_config(heads=4, kv_heads=2)
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=30, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        tok = tokens_for(cfg, 2 * cfg.seq + 1, seed=31)
        st.opt.zero_grads()
        for call in range(2):  # store, then accumulate
            st.opt.forward_backward(tok[:-1], tok[1:], 2, cfg.seq, 256.0)
            fused = st.opt.grad_norm()
            dev = _device_grads(st.opt, cfg.nlayers)
            ref = np.sqrt(sum(float(np.sum(np.asarray(a, np.float64) ** 2)) for _, a, _ in _pairs(dev, dev)))
            print(f"call {call}: fused norm {fused:.7e} float64 {ref:.7e}", flush=True)
            assert abs(fused - ref) <= 1e-6 * ref
        st.opt.grad_arena()  # hands out the pointer: the next norm is a full pass
        full = st.opt.grad_norm()
        assert abs(fused - full) <= 1e-6 * full
    finally:
        st.close()


def test_gradient_norm_sees_writes_through_the_handed_out_arena():
    """Once hb_opt_grad_arena has handed out the raw pointer, a backward's
    per-tile sums of squares no longer stand for the arena: the caller may
    write through the pointer after the backward. The norm must include such
    a write (here 1e-3 added to every gradient element through the pointer)."""
    import ctypes as C
    import os
    import torch
    hip = C.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    D2D = 3  # hipMemcpyDeviceToDevice
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=32, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        tok = tokens_for(cfg, cfg.seq + 1, seed=33)
        st.opt.zero_grads()
        ptr, n = st.opt.grad_arena()
        st.opt.forward_backward(tok[:-1], tok[1:], 1, cfg.seq, 256.0)
        k.ctx.synchronize()
        buf = torch.empty(n, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        assert hip.hipMemcpy(buf.data_ptr(), ptr, 4 * n, D2D) == 0
        buf += 1e-3
        torch.cuda.synchronize()
        assert hip.hipMemcpy(ptr, buf.data_ptr(), 4 * n, D2D) == 0
        dev = _device_grads(st.opt, cfg.nlayers)
        ref = np.sqrt(sum(float(np.sum(np.asarray(a, np.float64) ** 2)) for _, a, _ in _pairs(dev, dev)))
        norm = st.opt.grad_norm()
        print(f"norm after the caller's write {norm:.7e}, float64 of the arena {ref:.7e}", flush=True)
        assert abs(norm - ref) <= 1e-6 * ref
    finally:
        st.close()


def _rel_max(a, b):
    a, b = np.asarray(a, np.float64).reshape(-1), np.asarray(b, np.float64).reshape(-1)
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


@pytest.mark.parametrize("softcap", [0.0, 0.5])
def test_forward_result_then_backward(softcap):
    """The reference's pair forward() -> ForwardResult -> backward()
    (full_model.rs:73-81, 345-483) through hb_train_forward / hb_train_backward:
    ForwardResult's fields against the oracle on the device's weights, and the
    pair's gradients equal to hb_forward_backward's bit for bit."""
    cfg = tiny_config(heads=4, kv_heads=2)
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=40, std=0.05 if softcap else 0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        S, V, d = cfg.seq, cfg.vocab, cfg.dim
        tok = tokens_for(cfg, S + 1, seed=41)
        ocfg, ow = oracle_cfg(cfg), _rounded_oracle_weights(w)
        ref = O.model_forward(ocfg, ow, tok[:-1], tok[1:], softcap=softcap)
        raw = O.model_forward(ocfg, ow, tok[:-1], tok[1:])["logits"]
        _, dref = OB.cross_entropy_fwd_bwd(ref["logits"], tok[1:], V, F32(1) / F32(S))
        _, rinv_ref = O.rmsnorm_channel_first(ref["x_prenorm_cf"], ow.gamma_final, d, S)
        st.opt.zero_grads()
        fwd = E.forward(cfg, k, None, tok[:-1], tok[1:], softcap=softcap)
        assert fwd.dlogits.shape == (S * V,) and fwd.rms_inv_final.shape == (S,)
        assert fwd.x_final.shape == (d * S,) and fwd.x_prenorm.shape == (d * S,)
        errs = {"loss": abs(fwd.loss - float(ref["loss"])) / float(ref["loss"]),
                "dlogits": _rel_max(fwd.dlogits, dref),
                "x_final": _rel_max(fwd.x_final, ref["x_final_cf"]),
                "x_prenorm": _rel_max(fwd.x_prenorm, ref["x_prenorm_cf"]),
                "rms_inv_final": _rel_max(fwd.rms_inv_final, rinv_ref)}
        if softcap:
            errs["logits_capped"] = _rel_max(fwd.logits_capped, np.tanh(raw * (F32(1) / F32(softcap))))
        else:
            assert fwd.logits_capped.size == 0
        print(f"softcap {softcap}: " + ", ".join(f"{n} {e:.2e}" for n, e in errs.items()), flush=True)
        assert errs.pop("loss") <= LOSS_RTOL
        assert max(errs.values()) <= 5e-3, errs
        E.backward(cfg, k, None, fwd, tok[:-1], softcap, 256.0, st)
        pair = _device_grads(st.opt, cfg.nlayers)
        with pytest.raises(hb.HipBridgeError) as e:  # one backward per kept forward
            E.backward(cfg, k, None, fwd, tok[:-1], softcap, 256.0, st)
        assert e.value.code == hb.HB_E_STATE
        st.opt.zero_grads()
        st.opt.forward_backward(tok[:-1], tok[1:], 1, S, 256.0)
        fused = _device_grads(st.opt, cfg.nlayers)
        for name, a, b in _pairs(pair, fused):
            np.testing.assert_array_equal(a, b, err_msg=name)
        with pytest.raises(hb.HipBridgeError) as e:  # hb_forward_backward keeps nothing
            st.opt.backward(256.0)
        assert e.value.code == hb.HB_E_STATE
    finally:
        st.close()


def test_backward_keeps_the_forwards_softcap():
    """An inference forward with another softcap between the pair (it sets the
    model's softcap to its own) leaves the backward unchanged: the kept logits
    were capped with the training forward's softcap (full_model.rs:234-239),
    so the backward's tanh derivative uses that one. A backward called with
    another softcap or other tokens than the forward's is refused."""
    cfg = tiny_config(heads=4, kv_heads=2)
    k = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=42, std=0.05)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    try:
        S = cfg.seq
        tok = tokens_for(cfg, S + 1, seed=43)
        st.opt.zero_grads()
        fwd = E.forward(cfg, k, None, tok[:-1], tok[1:], softcap=0.5)
        E.forward_ws(cfg, k, None, tok[:-1], tok[1:], softcap=0.0)
        with pytest.raises(ValueError):
            E.backward(cfg, k, None, fwd, tok[:-1], 0.0, 256.0, st)
        other = tok[:-1].copy()
        other[0] = (other[0] + 1) % cfg.vocab
        with pytest.raises(ValueError):
            E.backward(cfg, k, None, fwd, other, 0.5, 256.0, st)
        E.backward(cfg, k, None, fwd, tok[:-1], 0.5, 256.0, st)
        pair = _device_grads(st.opt, cfg.nlayers)
        st.opt.zero_grads()
        k.set_softcap(0.5)
        st.opt.forward_backward(tok[:-1], tok[1:], 1, S, 256.0)
        fused = _device_grads(st.opt, cfg.nlayers)
        for name, a, b in _pairs(pair, fused):
            np.testing.assert_array_equal(a, b, err_msg=name)
        # and the softcap matters here: without it the gradients differ
        st.opt.zero_grads()
        k.set_softcap(0.0)
        st.opt.forward_backward(tok[:-1], tok[1:], 1, S, 256.0)
        uncapped = _device_grads(st.opt, cfg.nlayers)
        assert any(not np.array_equal(a, b) for _, a, b in _pairs(pair, uncapped))
    finally:
        st.close()


def test_error_paths():
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    k2 = CompiledKernels.compile(cfg)
    w = ModelWeights.synthetic(cfg, seed=17, std=0.02)
    st = E.ModelOptState(k, E.TrainConfig(), weights=w)
    other = hb.Optimizer(k2.model, E.TrainConfig())
    try:
        tok = tokens_for(cfg, cfg.seq + 1, seed=1)
        for bad in (dict(loss_scale=0.0), dict(S=cfg.seq + 1)):
            S = bad.get("S", cfg.seq)
            t = np.resize(tok, S + 1)
            with pytest.raises(hb.HipBridgeError) as e:
                st.opt.forward_backward(t[:-1], t[1:], 1, S, bad.get("loss_scale", 256.0))
            assert e.value.code == hb.HB_E_INVALID
        # an optimizer of another model
        with pytest.raises(hb.HipBridgeError):
            hb.call("hb_forward_backward", k.model.handle, other.handle, tok.ctypes.data,
                    tok.ctypes.data, 1, cfg.seq, 256.0, None, None)
        # out-of-range ids are refused on the host
        bad_tok = tok[:-1].copy()
        bad_tok[3] = cfg.vocab
        with pytest.raises(hb.HipBridgeError):
            st.opt.forward_backward(bad_tok, tok[1:], 1, cfg.seq, 256.0)
    finally:
        other.close()
        st.close()
