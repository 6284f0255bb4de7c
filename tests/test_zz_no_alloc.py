"""The allocation-free dispatch (g5moe_dispatch_noalloc) against the workspace
dispatch (g5moe_dispatch) through the C ABI: counts, offsets, perm and inv_pos
bit for bit, on two calls in a row (the second smaller, so the scratch array
holds the first call's ranks), with out-of-range entries, and against the C
oracle's counting sort.  Sizes beyond the scratch are refused before any work."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from genet5_amd import _lib, ops

pytestmark = pytest.mark.gpu


def run_both(idx_np, n_experts, dev):
    N, k = idx_np.shape
    idx = torch.from_numpy(np.ascontiguousarray(idx_np, dtype=np.int32)).to(dev)
    shape = _lib.make_shape(N, 128, 128, n_experts, k, _lib.DTYPE_BF16)
    S = ops._stream(dev)
    outs = []
    for noalloc in (False, True):
        counts = torch.full((n_experts,), -7, dtype=torch.int32, device=dev)
        offsets = torch.full((n_experts + 1,), -7, dtype=torch.int32, device=dev)
        perm = torch.full((N * k,), -7, dtype=torch.int32, device=dev)
        inv_pos = torch.full((N * k,), -7, dtype=torch.int32, device=dev)
        if noalloc:
            _lib.call("g5moe_dispatch_noalloc", ops._ptr(idx), ops._ptr(counts),
                      ops._ptr(offsets), ops._ptr(perm), ops._ptr(inv_pos), ctypes.byref(shape), S)
        else:
            ws = ops.workspace(shape, dev)
            _lib.call("g5moe_dispatch", ops._ptr(idx), ops._ptr(counts), ops._ptr(offsets),
                      ops._ptr(perm), ops._ptr(inv_pos), ops._ptr(ws), ctypes.byref(shape), S)
        outs.append((counts, offsets, perm, inv_pos))
    torch.cuda.synchronize()
    return outs


def test_noalloc_dispatch_equals_workspace_dispatch(cuda_device):
    rng = np.random.default_rng(17)
    cases = [(36400, 2, 16), (1000, 2, 16), (5000, 3, 7), (1, 1, 1)]
    for N, k, E in cases:
        print(f"noalloc dispatch N={N} k={k} E={E}", flush=True)
        idx = rng.integers(0, E, (N, k)).astype(np.int32)
        if N > 10:
            idx[rng.integers(0, N, 5), rng.integers(0, k, 5)] = -1  # not placed
            idx[rng.integers(0, N, 5), rng.integers(0, k, 5)] = E
        (c0, o0, p0, i0), (c1, o1, p1, i1) = run_both(idx, E, cuda_device)
        for a, b in ((c0, c1), (o0, o1), (p0, p1), (i0, i1)):
            assert torch.equal(a, b)
        counts, offsets, perm, inv_pos = oracle.dispatch_c(idx, E)
        placed = int(offsets[-1])
        np.testing.assert_array_equal(c1.cpu().numpy(), counts)
        np.testing.assert_array_equal(o1.cpu().numpy(), offsets)
        np.testing.assert_array_equal(p1.cpu().numpy()[:placed], perm[:placed])
        np.testing.assert_array_equal(i1.cpu().numpy(), inv_pos)


def test_noalloc_dispatch_refuses_beyond_its_scratch(cuda_device):
    k, E = 2, 16
    N = (1 << 20) // k + 1
    shape = _lib.make_shape(N, 128, 128, E, k, _lib.DTYPE_BF16)
    counts = torch.empty((E,), dtype=torch.int32, device=cuda_device)
    offsets = torch.empty((E + 1,), dtype=torch.int32, device=cuda_device)
    with pytest.raises(_lib.G5MoEError, match="exceeds its scratch") as ei:
        _lib.call("g5moe_dispatch_noalloc", None, ops._ptr(counts), ops._ptr(offsets), None,
                  None, ctypes.byref(shape), ops._stream(cuda_device))
    assert ei.value.status == 2  # G5MOE_ERR_UNSUPPORTED
