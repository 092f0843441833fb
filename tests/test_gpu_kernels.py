"""Kernel-level parity on the GPU, through the C ABI (per-kernel entry points).

Each stage of the reference layer (RMSNorm -> sdpaFwd -> woFwd -> residual ->
RMSNorm -> ffnFused, layer.rs:684-806) is run on the device and compared with
the oracle on the same inputs. Inputs to fp16 kernels are rounded to fp16
before they reach the oracle, so the comparison measures the kernels' own
error (fp32 accumulate) rather than input rounding.
"""
import numpy as np
import pytest

import oracle as O
from rustane_amd import hip_bridge as hb
from rustane_amd.engine import CompiledKernels, ModelWeights
from tests._util import F32, f16_round, oracle_cfg, oracle_weights, tiny_config, to_dev

pytestmark = pytest.mark.gpu


def _gemm_case(gpu, M, N, K, seed):
    import torch
    rng = np.random.default_rng(seed)
    a = f16_round(rng.standard_normal((M, K)))
    b = f16_round(rng.standard_normal((N, K)))
    da, db = to_dev(a, torch.float16), to_dev(b, torch.float16)
    dc = torch.full((M, N), float("nan"), device="cuda")
    hb.call("hb_op_gemm_nt", gpu.handle, da.data_ptr(), db.data_ptr(), dc.data_ptr(), M, N, K)
    torch.cuda.synchronize()
    ref = a.astype(np.float64) @ b.astype(np.float64).T
    return dc.cpu().numpy(), ref


@pytest.mark.parametrize("M,N,K", [
    (64, 64, 64),        # 64x64 tiles, single K slice
    (37, 68, 192),       # ragged token and feature tails
    (1024, 2048, 256),   # 128x128 tiles
    (512, 16384, 128),   # 256x128 tiles, XCD remap with 256 tiles
    (300, 1540, 320),    # tails + non power-of-two tile count
    (512, 22016, 64),    # 192x256 tiles (8 waves of 96x64), partial last row tile
    (300, 12288, 128),   # 192x128 tiles (4 waves of 96x64), ragged tokens
    (4096, 4096, 128),   # 256x256 tiles
])
def test_gemm_nt_matches_float64(gpu, M, N, K):
    print(f"gemm M={M} N={N} K={K}", flush=True)
    c, ref = _gemm_case(gpu, M, N, K, seed=M + N + K)
    assert np.isfinite(c).all()
    err = np.abs(c - ref).max()
    # fp16 inputs are exact; fp32 accumulation over K terms of size ~1.
    assert err < 1e-4 * K, err


def test_gemm_nt_mfma_layout_one_hot(gpu):
    """A one-hot A row selects exactly one B row: catches any lane/register
    layout mistake in the MFMA fragments independently of rounding."""
    import torch
    M, N, K = 64, 64, 64
    a = np.zeros((M, K), F32)
    for i in range(M):
        a[i, (7 * i + 3) % K] = 1.0
    b = f16_round(np.random.default_rng(0).standard_normal((N, K)))
    dc = torch.zeros((M, N), device="cuda")
    # keep the device tensors referenced until the kernel has run
    da, db = to_dev(a, torch.float16), to_dev(b, torch.float16)
    hb.call("hb_op_gemm_nt", gpu.handle, da.data_ptr(), db.data_ptr(), dc.data_ptr(), M, N, K)
    torch.cuda.synchronize()
    expect = np.stack([b[:, (7 * i + 3) % K] for i in range(M)])
    np.testing.assert_array_equal(dc.cpu().numpy(), expect)


@pytest.mark.parametrize("dim", [512, 1536, 2560, 4096, 4100, 9000])
def test_rmsnorm_op_matches_oracle(gpu, dim):
    """Rows held in registers (dim a multiple of 1024, or up to 8 chunks of
    1024 with the last one partial: the 600M and 5B widths) and the two-pass
    form for wider rows."""
    import torch
    T = 37
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((T, dim)) * 3).astype(F32)
    g = (1 + 0.1 * rng.standard_normal(dim)).astype(F32)
    out = torch.empty((T, dim), dtype=torch.float16, device="cuda")
    rinv = torch.empty(T, device="cuda")
    dx, dg = to_dev(x), to_dev(g)
    hb.call("hb_op_rmsnorm", gpu.handle, dx.data_ptr(), dg.data_ptr(), T, dim, 1e-5,
            out.data_ptr(), rinv.data_ptr())
    torch.cuda.synchronize()
    ref, ref_r = O.rmsnorm_channel_first(x.T.reshape(-1), g, dim, T)
    got_r = rinv.cpu().numpy()
    # the kernel's fp32 sum of squares (per-thread chunks, then a block tree)
    # stays within 2e-6 of float64; the oracle's sequential fp32 sum drifts
    # with the row length (about 2e-6 of rms_inv at 9000)
    r64 = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1) + 1e-5)
    np.testing.assert_allclose(got_r, r64, rtol=2e-6)
    np.testing.assert_allclose(got_r, ref_r, rtol=2e-6 if dim <= 4100 else 1e-5)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref.reshape(dim, T).T, rtol=1e-3, atol=1e-3)


@pytest.fixture(scope="module")
def tiny(gpu):
    cfg = tiny_config()
    k = CompiledKernels.compile(cfg)
    k.ctx.set_stream(gpu.stream())
    w = ModelWeights.synthetic(cfg, seed=1234, std=0.02)
    k.ensure_weights(w)
    return cfg, k, w


def test_embedding_op_exact(tiny):
    import torch
    cfg, k, w = tiny
    tok = np.array([0, 5, cfg.vocab - 1, 17, 5], np.uint32)
    x = torch.empty((tok.size, cfg.dim), device="cuda")
    dtok = to_dev(tok)
    hb.call("hb_op_embedding", k.model.handle, dtok.data_ptr(), tok.size, x.data_ptr())
    torch.cuda.synchronize()
    ref = f16_round(O.embedding_forward(w.embed, cfg.dim, tok).reshape(tok.size, cfg.dim))
    np.testing.assert_array_equal(x.cpu().numpy(), ref)


def test_synthetic_init_is_bit_identical_to_host_upload(gpu):
    cfg = tiny_config()
    tok = np.arange(cfg.seq, dtype=np.uint32) * 7 % cfg.vocab
    a = CompiledKernels.compile(cfg)
    a.init_synthetic(77, 0.02)
    b = CompiledKernels.compile(cfg)
    b.ensure_weights(ModelWeights.synthetic(cfg, seed=77, std=0.02))
    la = np.empty((cfg.seq, cfg.vocab), F32)
    lb = np.empty_like(la)
    for kk, out in ((a, la), (b, lb)):
        hb.call("hb_forward", kk.model.handle, hb.ptr(tok), None, 1, cfg.seq, None, hb.ptr(out), None)
    np.testing.assert_array_equal(la, lb)


def _layer_inputs(cfg, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((cfg.seq, cfg.dim)) * 0.5).astype(F32)


def test_layer_ops_match_oracle(tiny):
    """sdpaFwd (QKV + RoPE + causal attention), woFwd + residual, ffnFused, each
    against the oracle on identical (fp16-rounded) inputs."""
    import torch
    cfg, k, w = tiny
    oc = oracle_cfg(cfg)
    lw = oracle_weights(w).layers[0]
    S = cfg.seq
    x = _layer_inputs(cfg, 3)
    # RMSNorm1 on the device, then feed the same fp16 xnorm to both sides.
    dx = to_dev(x)
    dxn = torch.empty((S, cfg.dim), dtype=torch.float16, device="cuda")
    g1 = to_dev(lw.gamma1)
    hb.call("hb_op_rmsnorm", k.ctx.handle, dx.data_ptr(), g1.data_ptr(), S, cfg.dim, 1e-5,
            dxn.data_ptr(), None)
    dattn = torch.empty((S, cfg.q_dim), dtype=torch.float16, device="cuda")
    tap = torch.empty((S, cfg.q_dim + 2 * cfg.kv_dim), device="cuda")
    hb.call("hb_op_sdpa_fwd", k.model.handle, 0, dxn.data_ptr(), 1, S, dattn.data_ptr(), tap.data_ptr())
    torch.cuda.synchronize()
    xn = dxn.float().cpu().numpy()
    # weights as the device holds them (fp16)
    r = lambda a: f16_round(a)
    s = O.sdpa_fwd(oc, xn.T, r(lw.wq), r(lw.wk), r(lw.wv), S)
    t = tap.cpu().numpy()
    q, kv = cfg.q_dim, cfg.kv_dim
    np.testing.assert_allclose(t[:, :q], s["q_rope"].T, atol=2e-3)
    np.testing.assert_allclose(t[:, q:q + kv], s["k_rope"].T, atol=2e-3)
    np.testing.assert_allclose(t[:, q + kv:], s["v"].T, atol=2e-3)
    np.testing.assert_allclose(dattn.float().cpu().numpy(), s["attn"].T, atol=3e-3)

    # woFwd + residual on the device's own attn output
    attn = dattn.float().cpu().numpy()
    dx2 = torch.empty((S, cfg.dim), device="cuda")
    hb.call("hb_op_wo_fwd", k.model.handle, 0, dattn.data_ptr(), dx.data_ptr(), S, dx2.data_ptr())
    torch.cuda.synchronize()
    o = O.dyn_matmul(attn.T, r(lw.wo), cfg.q_dim, cfg.dim, S)
    x2 = O.vsma(o.reshape(-1), oc.alpha(), x.T.reshape(-1)).reshape(cfg.dim, S).T
    np.testing.assert_allclose(dx2.cpu().numpy(), x2, atol=1e-4)

    # ffnFused on a device-normed x2
    dx2n = torch.empty((S, cfg.dim), dtype=torch.float16, device="cuda")
    g2 = to_dev(lw.gamma2)
    hb.call("hb_op_rmsnorm", k.ctx.handle, dx2.data_ptr(), g2.data_ptr(), S, cfg.dim, 1e-5,
            dx2n.data_ptr(), None)
    dnext = torch.empty((S, cfg.dim), device="cuda")
    dh13 = torch.empty((S, 2 * cfg.hidden), device="cuda")
    dgate = torch.empty((S, cfg.hidden), dtype=torch.float16, device="cuda")
    hb.call("hb_op_ffn_fused", k.model.handle, 0, dx2n.data_ptr(), dx2.data_ptr(), S,
            dnext.data_ptr(), dh13.data_ptr(), dgate.data_ptr())
    torch.cuda.synchronize()
    x2n = dx2n.float().cpu().numpy()
    x2d = dx2.cpu().numpy()
    f = O.ffn_fused(oc, x2n.T, x2d.T, r(lw.w1), r(lw.w3), r(lw.w2), S)
    h13 = dh13.cpu().numpy()
    np.testing.assert_allclose(h13[:, :cfg.hidden], f["h1"].T, atol=1e-3)
    np.testing.assert_allclose(h13[:, cfg.hidden:], f["h3"].T, atol=1e-3)
    np.testing.assert_allclose(dgate.float().cpu().numpy(), f["gate"].T, atol=1e-3)
    # x_next from the device gate (fp16) vs oracle recomputed on that gate
    gate = dgate.float().cpu().numpy()
    ffn = gate @ r(lw.w2).reshape(cfg.dim, cfg.hidden).T
    np.testing.assert_allclose(dnext.cpu().numpy(), x2d + oc.alpha() * ffn, atol=1e-4)


def test_sdpa_op_on_staged_rope_tiles_spanning_sequences(gpu):
    """sdpaFwd for 3 sequences of 700 tokens on a 2048d / 16x128 model: the
    QKV GEMM then runs 256x256 tiles (216 of them, the launcher's choice for
    N = 6144, T = 2100), which copy their RoPE table slice into LDS per tile
    and read it from there. 700 is not a multiple of 256, so tiles hold the
    end of one sequence and the start of the next: each staged token must
    get its own position. Every sequence is checked against the oracle run
    alone."""
    import torch
    cfg = tiny_config(dim=2048, hidden=256, heads=16, hd=128, nlayers=1, seq=700, vocab=256)
    k = CompiledKernels.compile(cfg)
    k.ctx.set_stream(gpu.stream())
    w = ModelWeights.synthetic(cfg, seed=77, std=0.02)
    k.ensure_weights(w)
    oc = oracle_cfg(cfg)
    lw = oracle_weights(w).layers[0]
    B, S = 3, cfg.seq
    xn = f16_round(np.random.default_rng(11).standard_normal((B * S, cfg.dim)) * 0.5)
    dxn = to_dev(xn, torch.float16)
    dattn = torch.empty((B * S, cfg.q_dim), dtype=torch.float16, device="cuda")
    tap = torch.empty((B * S, cfg.q_dim + 2 * cfg.kv_dim), device="cuda")
    hb.call("hb_op_sdpa_fwd", k.model.handle, 0, dxn.data_ptr(), B, S, dattn.data_ptr(), tap.data_ptr())
    torch.cuda.synchronize()
    t, attn = tap.cpu().numpy(), dattn.float().cpu().numpy()
    q, kv = cfg.q_dim, cfg.kv_dim
    for b in range(B):
        rows = slice(b * S, (b + 1) * S)
        s = O.sdpa_fwd(oc, xn[rows].T, f16_round(lw.wq), f16_round(lw.wk), f16_round(lw.wv), S)
        print(f"sequence {b}: max|dq| {np.abs(t[rows, :q] - s['q_rope'].T).max():.2e} "
              f"max|dattn| {np.abs(attn[rows] - s['attn'].T).max():.2e}", flush=True)
        np.testing.assert_allclose(t[rows, :q], s["q_rope"].T, atol=2e-3)
        np.testing.assert_allclose(t[rows, q:q + kv], s["k_rope"].T, atol=2e-3)
        np.testing.assert_allclose(t[rows, q + kv:], s["v"].T, atol=2e-3)
        np.testing.assert_allclose(attn[rows], s["attn"].T, atol=3e-3)
    k.model.close()
    k.ctx.close()


@pytest.mark.parametrize("B,S", [(3, 700), (1, 512), (2, 100)])
def test_sdpa_plain_stores_equal_tapped(gpu, B, S):
    """The QKV GEMM's plain epilogue (no tap: Q, K and V^T addressed per
    token and per 32-feature block) and its tapped one (the fp32 tap too,
    addressed per quad) must write the same fp16 Q, K and V^T: the attention
    output is compared bit for bit, on several tile shapes (256x256 staged
    tiles at 3 x 700 tokens, smaller ones below)."""
    import torch
    cfg = tiny_config(dim=2048, hidden=256, heads=16, hd=128, nlayers=1, seq=S, vocab=256)
    k = CompiledKernels.compile(cfg)
    k.ctx.set_stream(gpu.stream())
    w = ModelWeights.synthetic(cfg, seed=78, std=0.02)
    k.ensure_weights(w)
    xn = f16_round(np.random.default_rng(12).standard_normal((B * S, cfg.dim)) * 0.5)
    dxn = to_dev(xn, torch.float16)
    plain = torch.empty((B * S, cfg.q_dim), dtype=torch.float16, device="cuda")
    tapped = torch.empty_like(plain)
    tap = torch.empty((B * S, cfg.q_dim + 2 * cfg.kv_dim), device="cuda")
    print(f"sdpa plain vs tapped: B={B} S={S}", flush=True)
    hb.call("hb_op_sdpa_fwd", k.model.handle, 0, dxn.data_ptr(), B, S, plain.data_ptr(), None)
    hb.call("hb_op_sdpa_fwd", k.model.handle, 0, dxn.data_ptr(), B, S, tapped.data_ptr(), tap.data_ptr())
    torch.cuda.synchronize()
    a, b = plain.cpu().numpy(), tapped.cpu().numpy()
    assert np.isfinite(a.astype(F32)).all()
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), np.abs(a.astype(F32) - b.astype(F32)).max()
    k.model.close()
    k.ctx.close()


def test_logits_ce_op_matches_oracle(tiny):
    import torch
    cfg, k, w = tiny
    T = 33
    rng = np.random.default_rng(5)
    xf = f16_round(rng.standard_normal((T, cfg.dim)))
    tgt = rng.integers(0, cfg.vocab, T).astype(np.uint32)
    dl = torch.empty((T, cfg.vocab), device="cuda")
    dloss = torch.empty(T, device="cuda")
    dxf, dtgt = to_dev(xf, torch.float16), to_dev(tgt)
    hb.call("hb_op_logits_ce", k.model.handle, dxf.data_ptr(), dtgt.data_ptr(), T, dl.data_ptr(),
            dloss.data_ptr())
    torch.cuda.synchronize()
    E = f16_round(w.embed)
    ref = O.sgemm_at(xf, T, cfg.dim, E, cfg.vocab, np.zeros(T * cfg.vocab, F32))
    np.testing.assert_allclose(dl.cpu().numpy(), ref, atol=2e-4)
    _, losses = O.cross_entropy_batch(dl.cpu().numpy(), tgt, cfg.vocab)
    np.testing.assert_allclose(dloss.cpu().numpy(), losses, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("vocab", [8192, 32000])
def test_cross_entropy_wide_vocab_matches_oracle(gpu, vocab):
    """Cross-entropy at the workloads' vocabulary sizes: each thread walks its
    row in batches of 8 float4 (32000 = 31.25 x 1024: the last batch is
    partial) and raises its running maximum between batches. Rows range from
    all-zero logits (loss = ln(vocab)) to logits of std ~30 (a few terms carry
    the sum); losses against the oracle's on the device's own logits."""
    import torch
    cfg = tiny_config(dim=64, hidden=64, heads=1, nlayers=1, vocab=vocab)
    k = CompiledKernels.compile(cfg)
    k.ctx.set_stream(gpu.stream())
    w = ModelWeights.synthetic(cfg, seed=11, std=0.02)
    k.ensure_weights(w)
    T = 48
    rng = np.random.default_rng(9)
    scale = np.array([0.0] * 4 + [1.0] * 12 + [30.0] * 16 + [200.0] * 16, F32)[:, None]
    xf = f16_round(rng.standard_normal((T, cfg.dim)) * scale)
    tgt = rng.integers(0, vocab, T).astype(np.uint32)
    tgt[-1] = vocab - 1
    dl = torch.empty((T, vocab), device="cuda")
    dloss = torch.empty(T, device="cuda")
    dxf, dtgt = to_dev(xf, torch.float16), to_dev(tgt)
    hb.call("hb_op_logits_ce", k.model.handle, dxf.data_ptr(), dtgt.data_ptr(), T, dl.data_ptr(),
            dloss.data_ptr())
    torch.cuda.synchronize()
    got = dloss.cpu().numpy()
    _, ref = O.cross_entropy_batch(dl.cpu().numpy(), tgt, vocab)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(got[:4], np.log(vocab), rtol=1e-6)
    assert np.isfinite(got).all()
    k.model.close()
    k.ctx.close()


def test_cross_entropy_out_of_range_target_is_nan_and_reported(gpu):
    """A target id >= vocab reaching the device: its row's loss is NaN, the
    other rows are unchanged, and the next synchronisation reports the target
    (error word bit 2) and clears it."""
    import torch
    cfg = tiny_config(dim=64, hidden=64, heads=1, nlayers=1, vocab=320)
    k = CompiledKernels.compile(cfg)
    k.ctx.set_stream(gpu.stream())
    k.ensure_weights(ModelWeights.synthetic(cfg, seed=5, std=0.02))
    T = 6
    rng = np.random.default_rng(4)
    xf = f16_round(rng.standard_normal((T, cfg.dim)))
    tgt = rng.integers(0, cfg.vocab, T).astype(np.uint32)
    tgt[2] = cfg.vocab
    tgt[4] = 0xFFFFFFFF
    dl = torch.empty((T, cfg.vocab), device="cuda")
    dloss = torch.empty(T, device="cuda")
    dxf, dtgt = to_dev(xf, torch.float16), to_dev(tgt)
    hb.call("hb_op_logits_ce", k.model.handle, dxf.data_ptr(), dtgt.data_ptr(), T, dl.data_ptr(),
            dloss.data_ptr())
    with pytest.raises(hb.HipBridgeError) as e:
        k.ctx.synchronize()
    assert e.value.code == hb.HB_E_INVALID and "target" in str(e.value)
    k.ctx.synchronize()  # the error word was cleared
    got = dloss.cpu().numpy()
    assert np.isnan(got[[2, 4]]).all()
    ok = [0, 1, 3, 5]
    _, ref = O.cross_entropy_batch(dl.cpu().numpy()[ok], tgt[ok], cfg.vocab)
    np.testing.assert_allclose(got[ok], ref, rtol=1e-5, atol=1e-5)
    k.model.close()
    k.ctx.close()


@pytest.mark.parametrize("T", [128, 200])
def test_residual_gemm_split_k_matches_float64(gpu, T):
    """Wo of a 2048-wide model at <= 256 tokens has few output tiles and a long
    K, so the residual GEMM splits K (4 ways at 128 tokens) and reduces the
    fp32 partials in split order before the residual epilogue. Checked against
    float64 on fp16-exact inputs, and repeat launches must agree bit for bit."""
    import torch
    from rustane_amd.engine import ModelConfig
    cfg = ModelConfig.make(dim=2048, hidden=256, heads=16, nlayers=1, seq=T, vocab=256, hd=128)
    k = CompiledKernels.compile(cfg)
    k.ctx.set_stream(gpu.stream())
    w = ModelWeights.synthetic(cfg, seed=3, std=0.02)
    k.ensure_weights(w)
    print(f"split-K Wo: T={T} N={cfg.dim} K={cfg.q_dim}", flush=True)
    rng = np.random.default_rng(T)
    attn = f16_round(rng.standard_normal((T, cfg.q_dim)))
    x = rng.standard_normal((T, cfg.dim)).astype(F32)
    dattn, dx = to_dev(attn, torch.float16), to_dev(x)
    outs = []
    for _ in range(2):
        dx2 = torch.empty((T, cfg.dim), device="cuda")
        hb.call("hb_op_wo_fwd", k.model.handle, 0, dattn.data_ptr(), dx.data_ptr(), T, dx2.data_ptr())
        torch.cuda.synchronize()
        outs.append(dx2.cpu().numpy())
    wo = f16_round(oracle_weights(w).layers[0].wo).reshape(cfg.q_dim, cfg.dim)
    alpha = oracle_cfg(cfg).alpha()
    ref = x.astype(np.float64) + alpha * (attn.astype(np.float64) @ wo.astype(np.float64))
    err = np.abs(outs[0] - ref).max()
    print(f"max|err| {err:.2e}", flush=True)
    assert err < 1e-4
    np.testing.assert_array_equal(outs[0], outs[1])
