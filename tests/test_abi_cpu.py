"""CPU-side checks of the C ABI and the host wrappers: the library loads, exports
every symbol include/g5moe.h declares, validates arguments before touching the
GPU, and the Python layer refuses to run anywhere but on a GPU."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from genet5_amd import _lib, ops
from genet5_amd.moe import MoEFeedForward

HEADER = Path(__file__).resolve().parent.parent / "include" / "g5moe.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g5moe_[a-z_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(g5lib):
    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(g5lib, n), n
    assert set(names) == set(_lib.EXPORTED)


def test_version(g5lib):
    v = g5lib.g5moe_version()
    assert v >> 16 == _lib.ABI_MAJOR == 2


def shape(**kw):
    base = dict(n_tokens=36400, d_model=768, d_ff=3072, n_experts=16, top_k=2, x_dtype=0)
    base.update(kw)
    return _lib.make_shape(**base)


def status_of(fn, *args):
    st = getattr(_lib.lib(), fn)(*args)
    return st, _lib.lib().g5moe_last_error().decode()


def test_workspace_size_layout(g5lib):
    s = shape()
    n = _lib.workspace_size(s)
    nk = 36400 * 2
    a = lambda v: (v + 255) // 256 * 256
    nblk = (nk + 255) // 256
    # h carries 384 rows after its last row: one 256-row GEMM tile of padding, and
    # the weight gradient's sorted-order slack (ops.H_SLACK)
    assert ops.H_SLACK == 384
    assert n == (a(0) + a(nblk * 16 * 4) + a(nk * 4) + a((nk + 384) * 3072 * 2) + a(nk * 768 * 2)
                 + a((36400 + 3) // 4 * 16 * 4))
    n32 = _lib.workspace_size(shape(x_dtype=1))
    assert n32 == n + a(36400 * 768 * 2)
    assert ops._h_offset(s) == a(0) + a(nblk * 16 * 4) + a(nk * 4)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(d_model=640), 2, "d_model"),
    (dict(d_model=64), 2, "d_model"),
    (dict(d_ff=100), 2, "d_ff"),
    (dict(n_experts=17), 2, "n_experts"),
    (dict(n_experts=0), 2, "n_experts"),
    (dict(top_k=5), 2, "top_k"),
    (dict(top_k=3, n_experts=2), 2, "top_k"),
    (dict(x_dtype=7), 1, "x_dtype"),
    (dict(n_tokens=-1), 1, "n_tokens"),
    (dict(n_tokens=2 ** 31), 2, "int32"),
    (dict(n_tokens=2 ** 22), 2, "4 GiB"),
])
def test_invalid_shapes_rejected(g5lib, kw, code, msg):
    n = ctypes.c_size_t(0)
    st, err = status_of("g5moe_workspace_size", ctypes.byref(shape(**kw)), ctypes.byref(n))
    assert st == code and msg in err


def test_reserved_must_be_zero(g5lib):
    s = shape()
    s.reserved = 1
    n = ctypes.c_size_t(0)
    st, err = status_of("g5moe_workspace_size", ctypes.byref(s), ctypes.byref(n))
    assert st == 1 and "reserved" in err


def test_null_pointers_rejected_before_any_gpu_work(g5lib):
    s = shape(n_tokens=8)
    st, err = status_of("g5moe_router_topk", None, None, None, None, None, None,
                        ctypes.byref(s), None)
    assert st == 1 and "x is NULL" in err
    st, err = status_of("g5moe_forward", *([None] * 13), ctypes.byref(s), None)
    assert st == 1 and "NULL" in err
    st, err = status_of("g5moe_combine", None, None, None, None, ctypes.byref(s), None)
    assert st == 1
    st, err = status_of("g5moe_dispatch", None, None, None, None, None, None, None, None)
    assert st == 1 and "shape is NULL" in err


def test_error_is_raised_as_exception(g5lib):
    with pytest.raises(_lib.G5MoEError, match="UNSUPPORTED.*d_model"):
        _lib.workspace_size(shape(d_model=100))


def test_wrappers_refuse_cpu_tensors():
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    w = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        ops.router_topk(x, w, 2)
    m = MoEFeedForward(128, 128, num_experts=4, top_k=2).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        m(torch.zeros(2, 3, 128, dtype=torch.bfloat16))


def test_module_constructor_contract():
    m = MoEFeedForward(768, 3072, 0.0)  # positional like lib/blocks/encoder.py:69
    assert m.w_gate.shape == (16, 3072, 768) and m.w_down.shape == (16, 768, 3072)
    assert m.router.weight.shape == (16, 768) and m.top_k == 2
    with pytest.raises(ValueError, match="silu"):
        MoEFeedForward(768, 3072, 0.0, "gelu_new")
    with pytest.raises(ValueError):
        MoEFeedForward(768, 3000)
    with pytest.raises(ValueError):
        MoEFeedForward(768, 3072, num_experts=4, top_k=5)
    # dropout in training mode runs the training path (bf16 activations, GPU only;
    # no CPU fallback)
    m.train()
    m.dropout = 0.1
    with pytest.raises(TypeError, match="bf16"):
        m(torch.zeros(1, 768))
    with pytest.raises(RuntimeError, match="GPU only"):
        m.to(torch.bfloat16)(torch.zeros(1, 768, dtype=torch.bfloat16))


def test_module_load_dense_upcycles():
    m = MoEFeedForward(128, 256, num_experts=4)
    wi0, wi1, wo = torch.randn(256, 128), torch.randn(256, 128), torch.randn(128, 256)
    m.load_dense(wi0, wi1, wo)
    for e in range(4):
        assert torch.equal(m.w_gate[e], wi0) and torch.equal(m.w_up[e], wi1)
        assert torch.equal(m.w_down[e], wo)


def test_fake_impl_traces_shape():
    from torch._subclasses.fake_tensor import FakeTensorMode
    from genet5_amd.moe import _moe_forward_op
    with FakeTensorMode():
        x = torch.empty(10, 768, dtype=torch.bfloat16)
        y = _moe_forward_op(x, torch.empty(16, 768, dtype=torch.bfloat16), None,
                            torch.empty(16, 6144, 768, dtype=torch.bfloat16),
                            torch.empty(16, 768, 3072, dtype=torch.bfloat16), 2)
        assert y.shape == x.shape and y.dtype == x.dtype


def test_training_op_fake_impl_shapes():
    """The training op's fake implementation (torch.compile traces it) gives the
    real op's ten outputs: y, logits, routing, y_perm, the SwiGLU operand for the
    backward [N*k, 2F] and the forward's h with its 384 slack rows; the backward
    op's fake gives one gradient per differentiable input, in its dtype."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from genet5_amd.moe import _moe_backward_op, _moe_forward_train_op
    N, d, F, E, k = 10, 768, 3072, 16, 2
    with FakeTensorMode():
        b = dict(dtype=torch.bfloat16)
        f = dict(dtype=torch.float32)
        x = torch.empty(N, d, **b)
        wr = torch.empty(E, d, **b)
        wg, wu, wd = torch.empty(E, F, d, **f), torch.empty(E, F, d, **f), torch.empty(E, d, F, **f)
        outs = _moe_forward_train_op(x, wr, None, wg, wu, wd, k, 0.1)
        shapes = [tuple(t.shape) for t in outs]
        assert outs[10].device.type == "cpu" and outs[10].dtype == torch.int64
        grads = _moe_backward_op(torch.empty(N, d, **b), None, x, wr, wg, wu, wd, *outs[2:10],
                                 k, 0.1, outs[10])
        gshapes = [(tuple(g.shape), g.dtype) for g in grads]
    assert shapes == [(N, d), (N, E), (N, k), (N, k), (E + 1,), (N * k,), (N * k,), (N * k, d),
                      (N * k, 2 * F), (N * k + ops.H_SLACK, F), (1,)]
    assert gshapes == [((N, d), torch.bfloat16), ((E, d), torch.bfloat16),
                       ((E, F, d), torch.float32), ((E, F, d), torch.float32),
                       ((E, d, F), torch.float32)]


@pytest.mark.parametrize("args,code,msg", [
    (dict(n=-1), 1, "n_rows"),
    (dict(dtype=3), 1, "dtype"),
    (dict(d=640), 2, "d_model"),
    (dict(eps=-1.0), 1, "eps"),
    (dict(sum_out=True), 1, "x_add"),
    (dict(), 1, "NULL"),
])
def test_rmsnorm_argument_checks(g5lib, args, code, msg):
    a = dict(n=4, d=768, dtype=0, eps=1e-6, sum_out=False)
    a.update(args)
    so = ctypes.c_void_p(0x1000) if a["sum_out"] else None
    st = g5lib.g5moe_rmsnorm(None, None, None, ctypes.c_float(a["eps"]), so, None, a["n"],
                             a["d"], a["dtype"], None)
    assert st == code and msg in g5lib.g5moe_last_error().decode()


def _wg_shape(d=768, F=3072):
    return _lib.make_shape(100, d, F, 16, 2, _lib.DTYPE_BF16)


@pytest.mark.parametrize("kw,code,msg", [
    (dict(kmax=200), 1, "multiple of 192"),
    (dict(kmax=192), 1, ">= 384"),
    (dict(F=384), 2, "multiples of 256"),
    (dict(d=128), 2, "multiples of 256"),
    (dict(), 1, "NULL"),
    (dict(misaligned=True), 2, "aligned"),
])
def test_weight_grad_argument_checks(g5lib, kw, code, msg):
    a = dict(kmax=384, d=768, F=3072, misaligned=False)
    a.update(kw)
    s = _wg_shape(a["d"], a["F"])
    p = ctypes.c_void_p(0x1000)
    bad = ctypes.c_void_p(0x1008)
    if a["misaligned"]:
        args = (p, bad, p, None, None, None, p)
    else:
        args = (None, None, p, None, None, None, None)   # an output without its operands
    st = g5lib.g5moe_weight_grad(*args, a["kmax"], ctypes.byref(s), None)
    assert st == code and msg in g5lib.g5moe_last_error().decode(), (st, g5lib.g5moe_last_error())


def test_weight_grad_and_pad_rows_nothing_to_do(g5lib):
    s = _wg_shape()
    # both outputs NULL: no work, no pointer touched
    assert g5lib.g5moe_weight_grad(None, None, None, None, None, None, None, 384,
                                   ctypes.byref(s), None) == 0
    assert g5lib.g5moe_weight_grad(None, None, None, None, None, None, None, 0,
                                   ctypes.byref(s), None) == 0


@pytest.mark.parametrize("cols,kmax,code,msg", [
    (12, 64, 1, "multiple of 8"),
    (768, -1, 1, "kmax"),
    (768, 64, 1, "NULL"),
    (768, 0, 1, "NULL"),  # kmax 0: the packed layout, which has rows to write
])
def test_pad_rows_argument_checks(g5lib, cols, kmax, code, msg):
    s = _wg_shape()
    st = g5lib.g5moe_pad_rows(None, None, None, None, cols, kmax, ctypes.byref(s), None)
    assert st == code and msg in g5lib.g5moe_last_error().decode()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(kmax=-1), 1, "kmax"),
    (dict(offsets=None), 1, "NULL"),
    (dict(dtype=_lib.DTYPE_F32), 2, "bf16"),
])
def test_gate_grad_padded_argument_checks(g5lib, kw, code, msg):
    a = dict(kmax=384, offsets=ctypes.c_void_p(0x1000), dtype=_lib.DTYPE_BF16)
    a.update(kw)
    s = _lib.make_shape(100, 768, 3072, 16, 2, a["dtype"])
    p = ctypes.c_void_p(0x1000)
    st = g5lib.g5moe_gate_grad_padded(p, p, p, p, a["offsets"], p, p, a["kmax"],
                                      ctypes.byref(s), None)
    assert st == code and msg in g5lib.g5moe_last_error().decode(), (st, g5lib.g5moe_last_error())
    # no tokens: the padded rows still get their zeros (384 per expert in the packed
    # layout), so offsets and dy_pad are needed, the token inputs are not
    s0 = _lib.make_shape(0, 768, 3072, 16, 2, _lib.DTYPE_BF16)
    assert g5lib.g5moe_gate_grad_padded(None, None, None, None, None, None, None, 0,
                                        ctypes.byref(s0), None) == 1
    assert "NULL" in g5lib.g5moe_last_error().decode()


def test_wgrad_kmax_rule():
    assert ops.wgrad_kmax(1) == 384 and ops.wgrad_kmax(384) == 384
    assert ops.wgrad_kmax(385) == 576 and ops.wgrad_kmax(5071) == 5184
    assert all(ops.wgrad_kmax(m) % 192 == 0 and ops.wgrad_kmax(m) >= m for m in range(0, 9000, 37))


def test_weight_grad_sorted_h_argument_checks(g5lib):
    s = _wg_shape()
    p = ctypes.c_void_p(0x1000)
    fn = g5lib.g5moe_weight_grad_sorted_h
    # gate without up (and the reverse)
    assert fn(None, None, None, p, p, p, None, p, 384, ctypes.byref(s), None) == 1
    assert "d_w_up is NULL" in g5lib.g5moe_last_error().decode()
    assert fn(None, None, None, p, p, None, p, p, 384, ctypes.byref(s), None) == 1
    assert "d_w_gate is NULL" in g5lib.g5moe_last_error().decode()
    # the down product without h
    assert fn(p, None, p, None, None, None, None, p, 384, ctypes.byref(s), None) == 1
    assert "h is NULL" in g5lib.g5moe_last_error().decode()
    assert fn(p, p, p, None, None, None, None, p, 200, ctypes.byref(s), None) == 1
    assert fn(p, p, p, None, None, None, ctypes.c_void_p(0x1008), p, 384, ctypes.byref(s),
              None) == 1
    # nothing requested: nothing done
    assert fn(None, None, None, None, None, None, None, None, 384, ctypes.byref(s), None) == 0


@pytest.mark.parametrize("n,chunks", [(0, 1), (1, 1), (64, 1), (65, 2), (36400, 256),
                                      (10 ** 6, 256)])
def test_router_weight_grad_scratch_size(g5lib, n, chunks):
    s = _lib.make_shape(n, 768, 3072, 16, 2, _lib.DTYPE_BF16)
    b = ctypes.c_size_t(0)
    assert g5lib.g5moe_router_weight_grad_scratch(ctypes.byref(s), ctypes.byref(b)) == 0
    assert b.value == chunks * 16 * 768 * 4


def test_router_weight_grad_argument_checks(g5lib):
    p = ctypes.c_void_p(0x1000)
    s = _lib.make_shape(10, 768, 3072, 16, 2, _lib.DTYPE_F32)
    assert g5lib.g5moe_router_weight_grad(p, p, p, p, ctypes.byref(s), None) == 2
    assert "bf16" in g5lib.g5moe_last_error().decode()
    s = _lib.make_shape(10, 768, 3072, 16, 2, _lib.DTYPE_BF16)
    assert g5lib.g5moe_router_weight_grad(None, p, p, p, ctypes.byref(s), None) == 1
    assert "dlogits is NULL" in g5lib.g5moe_last_error().decode()
    assert g5lib.g5moe_router_weight_grad(p, p, None, p, ctypes.byref(s), None) == 1
    assert g5lib.g5moe_router_weight_grad(p, ctypes.c_void_p(0x1004), p, p, ctypes.byref(s),
                                          None) == 2
    assert "aligned" in g5lib.g5moe_last_error().decode()
