"""Host-side checks of the C ABI and the engine mirror (no GPU needed).

The library must load, export exactly the entry points include/hip_bridge.h
declares, validate configs, generate the seeded synthetic inputs
deterministically, report failures through codes (including the injected
failure), and the Python mirror of rustane's engine API must match the
reference's presets and LCG init.
"""
import ctypes as C
import math
import os
import re

import numpy as np
import pytest

from rustane_amd import engine as E
from rustane_amd import hip_bridge as hb

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hip_bridge.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hb_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    fns = header_functions()
    for required in ("hb_ctx_create", "hb_model_create", "hb_model_upload_layer",
                     "hb_model_upload_embed", "hb_forward", "hb_kv_create", "hb_prefill",
                     "hb_decode_step", "hb_last_error", "hb_backend_name"):
        assert required in fns


def test_library_exports_every_declared_symbol():
    L = C.CDLL(hb.LIB_PATH)
    missing = [f for f in header_functions() if not hasattr(L, f)]
    assert not missing, missing
    # and the binding covers the whole header
    assert sorted(hb.SIGNATURES) == header_functions()


def test_backend_name_and_no_device_errors():
    assert hb.backend_name() == "hip-gfx950"
    if hb.device_count() > 0:
        pytest.skip("a GPU is visible; the no-device path is not reachable")
    with pytest.raises(hb.HipBridgeError) as e:
        hb.Context(0)
    assert e.value.code == hb.HB_E_DEVICE


def _cfg_struct(**kw):
    cfg = E.ModelConfig.llama_48m()
    s = hb.config_struct(cfg)
    for k, v in kw.items():
        setattr(s, k, v)
    return s


def test_config_validate_fills_reference_defaults():
    s = _cfg_struct(rope_theta=0.0, norm_eps=0.0, residual_alpha=0.0)
    hb.call("hb_config_validate", C.byref(s))
    assert s.rope_theta == 10000.0
    assert abs(s.norm_eps - 1e-5) < 1e-12
    # layer.rs:698: 1/sqrt(2*nlayers) in f32
    assert s.residual_alpha == np.float32(1.0) / np.sqrt(np.float32(16.0))


@pytest.mark.parametrize("field,value", [
    ("hd", 96), ("q_dim", 1024), ("kv_dim", 100), ("dim", 520), ("hidden", 1000),
    ("vocab", 32001), ("heads", 0), ("kv_heads", 3), ("gqa_ratio", 2), ("softcap", -1.0),
])
def test_config_validate_rejects(field, value):
    s = _cfg_struct(**{field: value})
    with pytest.raises(hb.HipBridgeError) as e:
        hb.call("hb_config_validate", C.byref(s))
    assert e.value.code == hb.HB_E_CONFIG
    assert hb.last_error()


def test_reference_presets_validate():
    for name in ("gpt_karpathy", "gpt_1024", "target_600m", "target_800m", "target_1b",
                 "target_1_5b", "mha_28l", "llama_48m", "llama_600m", "llama_5b", "llama_7b"):
        s = hb.config_struct(getattr(E.ModelConfig, name)())
        hb.call("hb_config_validate", C.byref(s))


def test_presets_match_reference_model_rs():
    # crates/engine/src/model.rs:21-151
    k = E.ModelConfig.gpt_karpathy()
    assert (k.dim, k.hidden, k.heads, k.hd, k.seq, k.nlayers, k.vocab) == (768, 2048, 6, 128, 512, 6, 8192)
    t = E.ModelConfig.target_600m()
    assert (t.dim, t.hidden, t.heads, t.nlayers, t.q_dim) == (1536, 4096, 12, 20, 1536)
    m = E.ModelConfig.mha_28l()
    assert (m.dim, m.hidden, m.heads, m.seq, m.nlayers) == (1024, 3072, 8, 256, 28)
    # param_count (model.rs:109-114)
    c = E.ModelConfig.llama_7b()
    assert c.param_count() == 32 * (4 * 4096 ** 2 + 3 * 4096 * 11008) + 32000 * 4096 + 4096 * 65


def test_random_vec_matches_sequential_lcg():
    # layer.rs:404-413, evaluated step by step in Python integers
    for n, scale in ((1, 1.0), (37, 0.5), (5000, 0.02)):
        got = E.random_vec(n, scale)
        seed = 42 + n
        for i in range(n):
            seed = (seed * 6364136223846793005 + 1442695040888963407) % (1 << 64)
            r = np.float32(np.float32(seed >> 32) / np.float32(4294967295.0)) * np.float32(2.0) - np.float32(1.0)
            assert got[i] == np.float32(r * np.float32(scale)), (n, i)


def test_synthetic_inputs_are_deterministic_and_normal():
    a = hb.synth_normal(1234, 5, 1 << 20)
    b = hb.synth_normal(1234, 5, 1 << 20)
    np.testing.assert_array_equal(a, b)
    c = hb.synth_normal(1234, 6, 1 << 20)
    assert np.mean(a == c) < 1e-3
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 1e-4
    z = a.astype(np.float64) / 0.02
    assert abs(np.mean(z ** 4) - 3.0) < 0.25  # near-normal kurtosis (Irwin-Hall 8: 2.85)
    assert np.abs(z).max() < 5.0
    # prefix property: element i does not depend on n
    np.testing.assert_array_equal(hb.synth_normal(1234, 5, 100), a[:100])
    t = hb.synth_tokens(42, 0, 32000, 100000)
    assert t.min() >= 0 and t.max() < 32000
    assert abs(t.mean() - 16000) < 300


def test_error_codes_and_injection():
    with pytest.raises(hb.HipBridgeError) as e:
        hb.call("hb_synth_normal", 1, 2, 0.02, 10, None)
    assert e.value.code == hb.HB_E_INVALID
    hb.call("hb_debug_inject_error", 7)
    try:
        for fn, args in (("hb_synth_tokens", (1, 2, 10, 4, None)), ("hb_device_count", (C.byref(C.c_int()),)),
                         ("hb_config_validate", (C.byref(_cfg_struct()),))):
            with pytest.raises(hb.HipBridgeError) as e:
                hb.call(fn, *args)
            assert e.value.code == hb.HB_E_INJECTED
            assert "injected" in hb.last_error()
    finally:
        hb.call("hb_debug_inject_error", 0)
    hb.call("hb_synth_tokens", 1, 2, 10, 4, np.empty(4, np.uint32).ctypes.data)


def test_error_message_is_thread_local():
    import threading
    msgs = {}

    def worker(tag, code):
        try:
            s = _cfg_struct(hd=code)
            hb.call("hb_config_validate", C.byref(s))
        except hb.HipBridgeError:
            pass
        msgs[tag] = hb.last_error()

    ts = [threading.Thread(target=worker, args=(i, 96 + i)) for i in range(4)]
    [t.start() for t in ts]
    [t.join() for t in ts]
    for i in range(4):
        assert f"got {96 + i}" in msgs[i]


def test_learning_rate_matches_oracle():
    """hb_learning_rate (host fp32, full_model.rs:334-342) against the oracle:
    bit-identical through the warmup; within 2 ulp on the cosine part, where
    the C library's cosf and numpy's float32 cos may round differently."""
    import oracle.optimizer as OP
    from rustane_amd import engine as E
    tc, otc = E.TrainConfig(), OP.TrainConfig()
    for s in range(0, tc.warmup_steps):
        assert np.float32(hb.learning_rate(tc, s)) == OP.learning_rate(s, otc), s
    for s in range(tc.warmup_steps, tc.total_steps + 1, 37):
        a = np.float32(hb.learning_rate(tc, s)).view(np.int32)
        b = OP.learning_rate(s, otc).view(np.int32)
        assert abs(int(a) - int(b)) <= 2, s
    with pytest.raises(hb.HipBridgeError):
        hb.learning_rate(E.TrainConfig(warmup_steps=0), 1)


def test_training_entry_points_reject_null_arguments():
    """hb_forward_backward(_device) check their handles and id pointers before
    touching a device (no GPU needed)."""
    import ctypes as C
    lib = hb.lib()
    ids = (C.c_uint32 * 4)()
    for name in ("hb_forward_backward", "hb_forward_backward_device"):
        f = getattr(lib, name)
        f.restype = C.c_int
        for args in ((None, None, ids, ids), (C.c_void_p(1), None, ids, ids),
                     (C.c_void_p(1), C.c_void_p(1), None, ids), (C.c_void_p(1), C.c_void_p(1), ids, None)):
            rc = f(*args, C.c_int(1), C.c_int(4), C.c_float(256.0), None, None)
            assert rc == hb.HB_E_INVALID, (name, rc)
            assert b"null" in lib.hb_last_error()
