"""The persistent grouped GEMM (g5moe_grouped_gemm, the kernel of the down product
and the backward's dh / dX products) across its pipeline variants: two fragment
slots (k-steps not a multiple of 3), three slots with the third A stage in the
epilogue region (k-steps a multiple of 3, at least 6), 128- and 256-column tiles,
the n-half tail, 128-row tiles (launches whose rows give fewer than 1.5 full
256 x 256 tiles per CU), experts with no rows, partial last tiles and workgroups
that run many tiles in a row.

Two checks per case.  (1) Each expert launched alone gives the same bits as the
full launch: an output element's MFMA chain runs over k in one fixed order whatever
workgroup, tile slot, stage buffer or tile height computes it, so a stage that lands
in the wrong buffer, a stale refill or a skipped tile breaks equality (a small
expert's solo launch takes 128-row tiles where the full launch may take 256-row
ones).  (2) Every expert's rows
match a float32 torch product of the same bf16 operands (rtol = atol = 2e-2 on
unit-scale outputs)."""
import numpy as np
import pytest
import torch

from genet5_amd import ops

pytestmark = pytest.mark.gpu


def _offsets(counts, device):
    off = np.zeros(len(counts) + 1, np.int32)
    off[1:] = np.cumsum(counts)
    return off, torch.tensor(off, dtype=torch.int32, device=device)


@pytest.mark.parametrize("K,n_out,counts", [
    (384, 256, [40000, 0, 257, 9000]),         # nk = 6: shortest three-stage tile
    (384, 256, [100000, 0, 257, 9000]),        # 256-row tiles, solos of 257 / 9000: 128
    (576, 768, [0, 1, 255, 256, 4097, 30000]),  # nk = 9, three n-tiles, half tail
    (448, 256, [12000, 3, 700]),               # nk = 7: two fragment slots
    (128, 128, [5000, 0, 999]),                # nk = 2, 128-column tiles
    (3072, 768, [9000, 4551, 0, 311]),         # the down product's K
    (6144, 768, [2500, 1300]),                 # the dX product's K
])
def test_grouped_gemm_pipeline_variants(cuda_device, K, n_out, counts):
    print(f"case K={K} n_out={n_out} counts={counts}", flush=True)
    g = torch.Generator(device=cuda_device).manual_seed(K + n_out)
    E = len(counts)
    rows = int(sum(counts))
    off, t_off = _offsets(counts, cuda_device)
    a = torch.randn(rows + ops.ROW_PAD, K, device=cuda_device, generator=g).to(torch.bfloat16)
    b = (torch.randn(E, n_out, K, device=cuda_device, generator=g) / K ** 0.5).to(torch.bfloat16)
    c = ops.grouped_gemm(a, rows, t_off, b)
    for e in range(E):
        o0, o1 = int(off[e]), int(off[e + 1])
        if o1 == o0:
            continue
        m = o1 - o0
        a_e = torch.zeros(m + ops.ROW_PAD, K, dtype=torch.bfloat16, device=cuda_device)
        a_e[:m] = a[o0:o1]
        one = torch.tensor([0, m], dtype=torch.int32, device=cuda_device)
        alone = ops.grouped_gemm(a_e, m, one, b[e:e + 1].contiguous())
        assert torch.equal(alone, c[o0:o1]), f"expert {e} differs from its solo launch"
        ref = a[o0:o1].float() @ b[e].float().T
        torch.testing.assert_close(c[o0:o1].float(), ref, rtol=2e-2, atol=2e-2)
    torch.cuda.synchronize()


@pytest.mark.parametrize("d,counts", [
    (768, [569, 570, 0, 568, 1, 1200, 571, 569, 569, 570, 0, 569, 1139, 568, 568, 569]),
    (256, [569, 0, 4000, 1, 255, 256, 257, 1700]),
    (768, [4550, 4550]),                                   # the EP-8 shard: 2 experts
])
def test_small_m_down_two_per_cu_equals_grouped_gemm(cuda_device, d, counts):
    """The down product at small M (a DP-8 / EP-8 shard's rows) runs 128 x 128 tiles
    with two workgroups per CU (g5moe_expert_down), while g5moe_grouped_gemm takes
    one 128 x 256 workgroup per CU there: each output's MFMA chain runs over k in
    the same order whatever the tile shape, so y_perm must equal the grouped GEMM
    on the same h and w_down bit for bit, with empty experts and partial tiles."""
    import ctypes
    from genet5_amd import _lib
    F, k = 3072, 2
    E = len(counts)
    rows = int(sum(counts))
    assert rows % k == 0
    print(f"small-M down d={d} E={E} rows={rows}", flush=True)
    g = torch.Generator(device=cuda_device).manual_seed(rows + d)
    off, t_off = _offsets(counts, cuda_device)
    shape = _lib.make_shape(rows // k, d, F, E, k, _lib.DTYPE_BF16)
    ws = ops.workspace(shape, cuda_device)
    h = ws[ops._h_offset(shape):].view(torch.bfloat16)[:(rows + ops.ROW_PAD) * F].view(-1, F)
    h.copy_(torch.randn(rows + ops.ROW_PAD, F, device=cuda_device, generator=g)
            .to(torch.bfloat16))
    wd = (torch.randn(E, d, F, device=cuda_device, generator=g) / F ** 0.5).to(torch.bfloat16)
    y_perm = torch.empty(rows, d, dtype=torch.bfloat16, device=cuda_device)
    _lib.call("g5moe_expert_down", ops._ptr(t_off), ops._ptr(wd), ops._ptr(y_perm),
              ops._ptr(ws), ctypes.byref(shape), ops._stream(cuda_device))
    ref = ops.grouped_gemm(h[:rows + ops.ROW_PAD].contiguous(), rows, t_off, wd)
    torch.cuda.synchronize()
    assert torch.equal(y_perm, ref)
    e = int(np.argmax(counts))
    o0, o1 = int(off[e]), int(off[e + 1])
    torch.testing.assert_close(y_perm[o0:o1].float(), h[o0:o1].float() @ wd[e].float().T,
                               rtol=2e-2, atol=2e-2)


def test_xcd_balanced_launches_equal_the_first(cuda_device):
    """The gate|up launches of 8 x 32 workgroups split their tile list over the XCDs
    by shares the launcher adapts to each XCD's measured speed (xcd_balance.hip), so
    the tile -> workgroup mapping changes from call to call while the weights settle.
    Every tile's arithmetic is the same whichever workgroup runs it: 40 forwards at
    config 2, each synchronised so that its records reach the launcher, must equal
    the first call's output bit for bit (the inference gate|up and, through the
    training op, the factor-storing one)."""
    from genet5_amd import synth
    from test_gpu_parity import layer_tensors
    print("xcd-balanced gate|up: 40 forwards against the first", flush=True)
    x, wr, wgu, wd, b = layer_tensors(synth.make_config(2, seed=3), cuda_device)
    buf = ops.ForwardBuffers(x.shape[0], x.shape[1], wd.shape[2], wd.shape[0], 2, x.dtype,
                             cuda_device)
    y0 = ops.moe_forward(x, wr, wgu, wd, 2, bias=b, buffers=buf).clone()
    t0 = ops.moe_forward_train(x, wr, wgu, wd, 2, bias=b, return_h=True, factors=True)
    t0 = [t.clone() for t in t0]
    torch.cuda.synchronize()
    for i in range(40):
        y = ops.moe_forward(x, wr, wgu, wd, 2, bias=b, buffers=buf)
        torch.cuda.synchronize()
        assert torch.equal(y, y0), f"forward {i}"
        if i % 8 == 7:
            t = ops.moe_forward_train(x, wr, wgu, wd, 2, bias=b, return_h=True, factors=True)
            torch.cuda.synchronize()
            for a, r in zip(t, t0):
                assert torch.equal(a, r), f"training forward after {i}"


@pytest.mark.parametrize("M,K,N", [(1, 768, 128), (700, 768, 768), (36400, 768, 2304),
                                   (5000, 256, 4096), (0, 768, 768)])
def test_linear_one_expert_product(cuda_device, M, K, N):
    """ops.linear (the grouped GEMM as a one-expert product, the config-5 encoder's
    projections): within bf16 rounding of a float32 product; bit-identical whether A
    is read in place (padded storage) or copied into a padded buffer first."""
    print(f"linear M={M} K={K} N={N}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(cuda_device)
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(cuda_device)
    xp = ops.empty_row_padded(M, K, torch.bfloat16, cuda_device)
    xp.copy_(x)
    assert ops._has_row_pad(xp) and (M == 0 or not ops._has_row_pad(x))
    y1 = ops.linear(x, w)
    y2 = ops.linear(xp, w)
    torch.cuda.synchronize()
    assert y1.shape == (M, N) and torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    if M:
        ref = x.float() @ w.float().t()
        err = (y1.float() - ref).abs()
        # one bf16 rounding of an fp32 sum: |err| <= 2^-8 |ref| (plus fp32 order noise)
        assert (err <= ref.abs() * 2.0 ** -8 + 1e-3).all()


def test_linear_first_call_under_graph_capture(cuda_device):
    """ops.linear's first call for a row count made under HIP graph capture (its
    [0, M] offsets then exist only in the graph): every replay, with eager calls of
    the same shape between them, equals the eager product bit for bit."""
    print("linear under graph capture", flush=True)
    M, K, N = 1237, 768, 768
    g = torch.Generator(device="cpu").manual_seed(3)
    xp = ops.empty_row_padded(M, K, torch.bfloat16, cuda_device)
    xp.copy_(torch.randn(M, K, generator=g).to(torch.bfloat16))
    w = (torch.randn(N, K, generator=g) * 0.05).to(torch.bfloat16).to(cuda_device)
    assert (cuda_device, M) not in ops._ROW_OFFSETS
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(cuda_device)
    side.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            y = ops.linear(xp, w)
    torch.cuda.current_stream(cuda_device).wait_stream(side)
    assert (cuda_device, M) not in ops._ROW_OFFSETS
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        eager = ops.linear(xp, w)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), eager.view(torch.int16))
