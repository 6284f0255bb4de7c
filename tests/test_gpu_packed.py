"""The backward's packed padded layout (kmax = 0) against the kmax layout, bit for bit.

In the kmax layout expert e's padded rows start at e * kmax; in the packed layout
they start at the sum of R_e' = max(384, 192 ceil(M_e' / 192)) over e' < e, which
the kernels compute from offsets on the device, so the host needs no expert
counts (the buffers hold N k + 384 E rows).  Every entry point that takes the
layout gets the same inputs in both layouts: g5moe_gate_grad_padded (dw and dY),
g5moe_pad_rows (gathered x rows), g5moe_dh_swiglu_backward (dGU),
g5moe_grouped_gemm_padded (the dX product), g5moe_swiglu_backward (dGU and h),
g5moe_weight_grad and g5moe_weight_grad_sorted_h.  The R_e rows of each expert
must be equal bit for bit, the rows past the last expert's untouched, and the
products equal.  Counts include empty experts first and last, one-row experts,
counts on and just past the 192/384 steps, and an empty batch."""
import ctypes

import numpy as np
import pytest
import torch

from genet5_amd import _lib, ops, synth
from test_gpu_parity import dev_t

pytestmark = pytest.mark.gpu

CASES = [[0, 1, 192, 384, 385, 2000, 4100], [700, 3, 0, 0], [0, 0, 0], [3, 1]]


def rows_of(c):
    return max(384, 192 * -(-c // 192))


def layout(counts, kmax):
    """First row of each expert in the layout of kmax (0: packed), and the rows in all."""
    if kmax > 0:
        return [e * kmax for e in range(len(counts))], len(counts) * kmax
    starts, s = [], 0
    for c in counts:
        starts.append(s)
        s += rows_of(c)
    return starts, s


def same_rows(a, a_kmax, b, b_kmax, counts, what):
    """Each expert's R_e padded rows of buffer a (layout a_kmax) equal b's (b_kmax)."""
    sa, _ = layout(counts, a_kmax)
    sb, _ = layout(counts, b_kmax)
    for e, c in enumerate(counts):
        r = rows_of(c)
        assert torch.equal(a[sa[e]:sa[e] + r].view(torch.int16),
                           b[sb[e]:sb[e] + r].view(torch.int16)), (what, e)


@pytest.mark.parametrize("counts", CASES)
def test_packed_layout_equals_kmax_layout(cuda_device, counts):
    dev = cuda_device
    print(f"packed vs kmax layout: counts={counts}", flush=True)
    g = torch.Generator(device=dev).manual_seed(17)
    rng = np.random.default_rng(17)
    E, d, F, k = len(counts), 768, 512, 2
    counts = list(counts)
    if sum(counts) % k:
        counts[-1] += 1
    offsets = np.zeros(E + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    T = int(offsets[-1])
    n = T // k
    t_off = dev_t(offsets, dev)
    kmax = ops.wgrad_kmax(max(counts))
    P = ops.packed_rows(T, E)
    _, p_used = layout(counts, 0)
    assert p_used <= P
    shape = _lib.make_shape(n, d, F, E, k, _lib.DTYPE_BF16)
    S = ops._stream(dev)
    inv = rng.permutation(T).astype(np.int32)
    t_inv = dev_t(inv, dev)
    perm = dev_t(np.argsort(inv).astype(np.int32), dev)
    w = torch.tensor(rng.random((max(n, 1), k)).astype(np.float32), device=dev)[:n]
    dy = torch.randn(max(n, 1), d, device=dev, generator=g).to(torch.bfloat16)[:n].contiguous()
    y_perm = torch.randn(max(T, 1), d, device=dev, generator=g).to(torch.bfloat16)[:T].contiguous()
    x = torch.randn(max(n, 1), d, device=dev, generator=g).to(torch.bfloat16)[:n].contiguous()

    # gate gradient: dw and the padded dY
    bufs, dws = {}, {}
    for km, rows in ((kmax, E * kmax), (0, P)):
        buf = torch.full((rows + ops.ROW_PAD, d), -3.0, dtype=torch.bfloat16, device=dev)
        dw = torch.full((max(n, 1), k), 5.0, dtype=torch.float32, device=dev)
        _lib.call("g5moe_gate_grad_padded", ops._ptr(dy), ops._ptr(y_perm), ops._ptr(t_inv),
                  ops._ptr(w), ops._ptr(t_off), ops._ptr(dw), ops._ptr(buf), km,
                  ctypes.byref(shape), S)
        bufs[km], dws[km] = buf, dw
    torch.cuda.synchronize()
    assert torch.equal(dws[kmax].view(torch.int32), dws[0].view(torch.int32))
    same_rows(bufs[kmax], kmax, bufs[0], 0, counts, "dY")
    # rows past the last expert's: untouched
    assert torch.equal(bufs[0][p_used:], torch.full_like(bufs[0][p_used:], -3.0))

    # gathered x rows
    xk = ops.pad_rows(x, perm, t_off, E, kmax, k, n_assignments=T).view(E * kmax, d)
    x0 = ops.pad_rows(x, perm, t_off, E, 0, k, n_assignments=T)
    assert x0.shape == (P, d)
    torch.cuda.synchronize()
    same_rows(xk, kmax, x0, 0, counts, "x rows")

    # dh + SwiGLU backward into dGU
    wd_t = (torch.randn(E, F, d, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    fac = torch.randn(max(T, 1), 2 * F, device=dev, generator=g).to(torch.bfloat16)[:T]
    fac = fac.contiguous()
    dgus = {}
    for km, rows in ((kmax, E * kmax), (0, P)):
        dgu = torch.full((rows + ops.ROW_PAD, 2 * F), -7.0, dtype=torch.bfloat16, device=dev)
        _lib.call("g5moe_dh_swiglu_backward", ops._ptr(bufs[km]), km, ops._ptr(t_off),
                  ops._ptr(wd_t), ops._ptr(fac), ops._ptr(dgu), ctypes.byref(shape), S)
        dgus[km] = dgu
    torch.cuda.synchronize()
    same_rows(dgus[kmax], kmax, dgus[0], 0, counts, "dGU")

    # the dX product over either padded dGU
    wgu_t = (torch.randn(E, d, 2 * F, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    if T > 0:
        dx_k = ops.grouped_gemm_padded(dgus[kmax], kmax, T, t_off, wgu_t)
        dx_0 = ops.grouped_gemm_padded(dgus[0], 0, T, t_off, wgu_t)
        torch.cuda.synchronize()
        assert torch.equal(dx_k, dx_0)

    # staged SwiGLU backward: padded dGU and h in both layouts
    dh = torch.randn(max(T, 1), F, device=dev, generator=g).to(torch.bfloat16)[:T].contiguous()
    gu = torch.randn(max(T, 1), 2 * F, device=dev, generator=g).to(torch.bfloat16)[:T]
    gu = gu.contiguous()
    st = {}
    for km, rows in ((kmax, E * kmax), (0, P)):
        dgu_pad = torch.full((rows + ops.ROW_PAD, 2 * F), 9.0, dtype=torch.bfloat16, device=dev)
        h_pad = torch.full((rows, F), 9.0, dtype=torch.bfloat16, device=dev)
        _lib.call("g5moe_swiglu_backward", ops._ptr(dh), ops._ptr(gu), ops._ptr(perm),
                  ops._ptr(t_off), None, ops._ptr(h_pad), ops._ptr(dgu_pad), km, None,
                  ctypes.byref(shape), S)
        st[km] = (dgu_pad, h_pad)
    torch.cuda.synchronize()
    same_rows(st[kmax][0], kmax, st[0][0], 0, counts, "staged dGU")
    same_rows(st[kmax][1], kmax, st[0][1], 0, counts, "staged h")

    # weight gradients: padded h, and h in sorted order
    h = torch.zeros(T + ops.H_SLACK, F, dtype=torch.bfloat16, device=dev)
    h[:T] = torch.randn(T, F, device=dev, generator=g).to(torch.bfloat16)
    res = {}
    for km in (kmax, 0):
        dy_pad = bufs[km][:E * kmax if km else P]
        xp = xk if km else x0
        d_wd, d_wgu = ops.weight_grad(dy_pad.view(E, kmax, d) if km else dy_pad,
                                      st[km][1].view(E, kmax, F) if km else st[km][1],
                                      dgus[km][:E * kmax].view(E, kmax, 2 * F) if km
                                      else dgus[km][:P],
                                      xp.view(E, kmax, d) if km else xp, t_off, km, top_k=k)
        wd2 = torch.empty_like(d_wd)
        wg2 = torch.empty(E, F, d, dtype=torch.bfloat16, device=dev)
        wu2 = torch.empty_like(wg2)
        _lib.call("g5moe_weight_grad_sorted_h", ops._ptr(dy_pad), ops._ptr(h), ops._ptr(wd2),
                  ops._ptr(dgus[km]), ops._ptr(xp), ops._ptr(wg2), ops._ptr(wu2),
                  ops._ptr(t_off), km, ctypes.byref(shape), S)
        res[km] = (d_wd, d_wgu, wd2, wg2, wu2)
    torch.cuda.synchronize()
    for a, b in zip(res[kmax], res[0]):
        assert torch.equal(a, b)
    if T == 0:
        assert not any(t.any() for t in res[0])
