"""The allocation-free Wo entry point (hb_op_wo_fwd_noalloc) against the
allocating one (hb_op_wo_fwd) through the C ABI: bit-identical outputs on two
calls in a row, the second with fewer tokens (its split count and partial-sum
layout differ, and the shared scratch array keeps the first call's contents),
and no device memory allocated by it."""
import numpy as np
import pytest

from rustane_amd import hip_bridge as hb
from rustane_amd.engine import CompiledKernels, ModelConfig

pytestmark = pytest.mark.gpu


def test_wo_fwd_noalloc_equals_allocating_entry_point(gpu):
    import torch
    # one layer of the 7B shape: Wo [4096 x 4096], the split-K products the
    # 512-token forward runs (2 splits at 512 tokens, 4 at 200)
    cfg = ModelConfig.make(dim=4096, hidden=11008, heads=32, nlayers=1, seq=512, vocab=256)
    k = CompiledKernels.compile(cfg)
    k.init_synthetic(81)
    gen = torch.Generator(device="cuda").manual_seed(82)
    for T in (512, 200):
        print(f"no-alloc Wo: T={T}", flush=True)
        attn = (torch.randn(T, cfg.q_dim, device="cuda", generator=gen) * 0.5).to(torch.float16)
        x = torch.randn(T, cfg.dim, device="cuda", generator=gen)
        ref = torch.empty(T, cfg.dim, device="cuda")
        got = torch.full((T, cfg.dim), float("nan"), device="cuda")
        hb.call("hb_op_wo_fwd", k.model.handle, 0, attn.data_ptr(), x.data_ptr(), T, ref.data_ptr())
        k.ctx.synchronize()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        hb.call("hb_op_wo_fwd_noalloc", k.model.handle, 0, attn.data_ptr(), x.data_ptr(), T, got.data_ptr())
        k.ctx.synchronize()
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info()[0] == free0
        assert torch.equal(got, ref), float((got - ref).abs().max())
    with pytest.raises(hb.HipBridgeError) as e:
        hb.call("hb_op_wo_fwd_noalloc", k.model.handle, 1, attn.data_ptr(), x.data_ptr(), 200, got.data_ptr())
    assert e.value.code == hb.HB_E_STATE
