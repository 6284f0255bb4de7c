"""Committed golden vectors (tests/golden/, written by make_golden.py) for the
config-1 shape: the synthetic generator still produces the same inputs, the
oracle still produces the same routing bit for bit and the same outputs, and the
GPU kernels reproduce the routing exactly and the outputs within tolerance."""
import hashlib
from pathlib import Path

import numpy as np
import pytest

import oracle
from genet5_amd import synth

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = ["f32", "bf16"]


def load(dtype):
    return dict(np.load(GOLDEN / f"cfg1_{dtype}_seed0.npz", allow_pickle=False))


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("dtype", CASES)
def test_generator_and_oracle_reproduce_golden(dtype):
    g = load(dtype)
    inp = synth.make_layer(2048, seed=0, dtype=dtype)
    for name in ("x", "w_router", "w_gate", "w_up", "w_down"):
        assert digest(getattr(inp, name)) == str(g[f"sha_{name}"]), name
    ref = oracle.moe_forward(inp.x, inp.w_router, inp.w_gate, inp.w_up, inp.w_down, 2,
                             storage="bf16")
    np.testing.assert_array_equal(ref["topk_idx"], g["topk_idx"])
    np.testing.assert_array_equal(ref["counts"], g["counts"])
    np.testing.assert_array_equal(ref["offsets"], g["offsets"])
    np.testing.assert_array_equal(ref["perm"], g["perm"])
    np.testing.assert_array_equal(ref["inv_pos"], g["inv_pos"])
    np.testing.assert_allclose(ref["topk_w"], g["topk_w"], rtol=0, atol=1e-7)
    np.testing.assert_allclose(ref["y"][g["rows"]], g["y_rows"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(np.linalg.norm(ref["y"].astype(np.float64), axis=1),
                               g["y_row_norms"], rtol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", CASES)
def test_gpu_matches_golden(cuda_device, dtype):
    import torch
    from genet5_amd import ops
    g = load(dtype)
    inp = synth.make_layer(2048, seed=0, dtype=dtype)
    t = synth.to_torch(inp, cuda_device)
    wgu = ops.pack_gate_up(t["w_gate"], t["w_up"])
    y, r = ops.moe_forward(t["x"], t["w_router"], wgu, t["w_down"], 2, return_routing=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(r.topk_idx.cpu().numpy(), g["topk_idx"])
    np.testing.assert_array_equal(r.counts.cpu().numpy(), g["counts"])
    np.testing.assert_array_equal(r.offsets.cpu().numpy(), g["offsets"])
    np.testing.assert_array_equal(r.perm.cpu().numpy(), g["perm"])
    np.testing.assert_array_equal(r.inv_pos.cpu().numpy(), g["inv_pos"])
    np.testing.assert_allclose(r.topk_w.cpu().numpy(), g["topk_w"], atol=2e-6)
    yg = y.float().cpu().numpy()
    rows = g["y_rows"]
    err = np.abs(yg[g["rows"]] - rows).max() / np.abs(rows).max()
    assert err <= 2e-2, err
    norms = np.linalg.norm(yg.astype(np.float64), axis=1)
    assert np.abs(norms - g["y_row_norms"]).max() / g["y_row_norms"].max() <= 1e-2
