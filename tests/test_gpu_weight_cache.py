"""The expert weight cache of MoEFeedForward (genet5_amd.moe._ExpertWeightCache).

The module's forwards read bf16 packed copies of w_gate / w_up / w_down that are
kept between calls.  A copy must follow every change of its parameters:
an in-place update (an optimizer step bumps the version counter) rebuilds it
under the same key; replacing a parameter's storage (`p.data = ...`, as a
checkpoint loader does) gives a new key and must drop the old copy instead of
leaving it behind; freeing the module drops its copies.  Each output is compared
bit for bit with a freshly built module holding the same weights."""
import gc

import pytest
import torch

from genet5_amd import moe as moe_mod
from genet5_amd.moe import MoEFeedForward

pytestmark = pytest.mark.gpu


def _fresh_output(m, x):
    ref = MoEFeedForward(768, 3072, 0.0, num_experts=16, top_k=2).to(x.device)
    ref = ref.to(torch.bfloat16).eval()
    with torch.no_grad():
        ref.load_state_dict(m.state_dict())
        y = ref(x)
    del ref
    return y


def test_cache_follows_updates_and_storage_swaps(cuda_device):
    print("weight cache: in-place update, storage swap, free", flush=True)
    moe_mod.clear_weight_cache()
    torch.manual_seed(0)
    m = MoEFeedForward(768, 3072, 0.0, num_experts=16, top_k=2).to(cuda_device)
    m = m.to(torch.bfloat16).eval()
    x = torch.randn(3000, 768, device=cuda_device).to(torch.bfloat16)
    with torch.no_grad():
        y0 = m(x).clone()
        assert len(moe_mod._WEIGHTS._entries) == 1
        builds = moe_mod._WEIGHTS.builds
        m(x)
        assert moe_mod._WEIGHTS.builds == builds        # unchanged weights: no rebuild

        m.w_gate.add_(0.01)                              # in place: version bump
        y1 = m(x).clone()
        assert moe_mod._WEIGHTS.builds == builds + 1
        assert len(moe_mod._WEIGHTS._entries) == 1
        assert not torch.equal(y1, y0)
        assert torch.equal(y1, _fresh_output(m, x))

        m.w_up.data = m.w_up.data.clone() * 0.5          # new storage, same parameter
        y2 = m(x).clone()
        assert len(moe_mod._WEIGHTS._entries) == 1       # the stale copy was dropped
        assert torch.equal(y2, _fresh_output(m, x))
    torch.cuda.synchronize()
    del m
    gc.collect()
    assert len(moe_mod._WEIGHTS._entries) == 0
