"""CPU restatement of the MoE layer forward — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker.

Functions, what they follow, and what pins them (tests/test_oracle.py):

router_logits / router_logits_np
    logits[t, e] = sum_j x[t, j] * Wr[e, j] (+ b[e]) — nn.Linear(d, E,
    bias=False) in the orientation of lib/blocks/_component.py:42-44; the
    router itself is new (README.md:12).  Summation order is the one the C ABI
    fixes (include/g5moe.h, g5moe_router_topk).  router_logits is the C
    implementation (oracle/g5moe_oracle.c), router_logits_np an independent
    vectorised numpy restatement.  Pins: C == numpy bit for bit on bf16 inputs
    (products exact in fp32); both within fp32 rounding of a float64 matmul;
    exactly-representable sums (integer-valued inputs) equal the closed form;
    a permutation of the lane chunks that the order forbids changes bits.
topk_gates / topk_gates_c
    Top-k by an increasing-expert scan that replaces only on a strictly greater
    logit (ties -> lower index; slot 0 = largest); gates = softmax over all
    experts (float64), renormalised over the k chosen.  Pins: constructed ties,
    numpy argsort(-logits, stable) on tie-free rows, gates == closed form
    1 / (1 + exp(l1 - l0)) for k = 2, sum to 1, k = E and E = 1 cases.
dispatch / dispatch_c
    counts, exclusive offsets, perm = stable argsort of topk_idx.flatten(),
    inv_pos = its inverse.  Pins: pure-Python brute force on small inputs,
    numpy argsort(kind='stable'), bijection and per-token invariants.
expert_forward
    h = silu(X Wg^T) * (X Wu^T), y = h Wd^T per expert over its rows —
    FeedForward.forward (lib/blocks/_component.py:48-52, 'silu' at :31); with
    storage="bf16" h and y are rounded to bf16 where the bf16 dataflow stores
    them, and moe_forward rounds an fp32 x to bf16 on its way into the expert
    products (round_bf16 is pinned against torch's bf16 cast).  Pins:
    float64 brute force on tiny inputs; upcycling invariant (all experts equal
    one dense FeedForward => MoE output == dense output, since the k gates sum
    to 1); zero down weights => zero output; E = 1, k = 1 reduces to dense.
combine
    y[t] = sum_s w[t, s] * y_perm[inv_pos[t, s]], fp32, slot order.  Pins: a
    permutation-equivariance check (permuting tokens permutes y) and the
    upcycling invariant above.
combine_c
    The C restatement of the combine as the C ABI fixes it (fmaf in slot order
    from 0, one rounding to the activation dtype) and of the residual variant
    out = T(r + T(T(acc) * alpha)) — the encoder block's
    `hidden_states + ff_output * alpha` (lib/blocks/encoder.py:89).  Pins:
    exact-rational fma restatement; k = 1, w = 1 returns y_perm bit for bit;
    the residual composition equals torch's own bf16 ops (CPU) on y_moe.
input_grad_c
    The C restatement of g5moe_input_grad (dX_perm rows added in slot order,
    then fmaf over experts in order, one rounding).  Pins: an exact-rational
    restatement (each addition and fma rounded once to fp32) on small inputs,
    including skipped positions; with zero dlogits it is the slot sum.
moe_backward
    Float64 textbook backward of the layer for fixed routing indices: gate
    gradient dw = dy . Y, dY = w dy, dh = dY Wd_e, SwiGLU derivative
    dg = dh u s (1 + g (1 - s)), du = dh g s, dx = dg Wg_e + du Wu_e + dlogits Wr,
    dlogits through the renormalised top-k softmax w_r (dw_r - sum w dw), weight
    gradients as outer products.  Pins: central finite differences of a
    scalar loss in random directions (float64), and torch.autograd in float64
    on a torch restatement of the same forward.
dropout_keep / dropout_keep_py / dropout_scale
    The dropout mask on the expert hidden state as the C ABI defines it
    (g5moe_dropout in include/g5moe.h; the reference applies nn.Dropout to the
    SwiGLU output in training, lib/blocks/_component.py:45, :51, whose Philox
    stream is torch's own and not reproduced): for assignment a and h column f,
    key = fmix32(fmix32(a ^ seed_lo) + seed_hi), bits = fmix32(key + (f >> 1) *
    0x9e3779b9), keep = 16 bits of it (low for even f, high for odd) >= thr with
    thr = round(p * 65536), scale = 65536 / (65536 - thr).  fmix32 is
    MurmurHash3's 32-bit finalizer.  dropout_keep is vectorised numpy,
    dropout_keep_py a pure-Python integer restatement.  Pins
    (tests/test_oracle_dropout.py): numpy == pure Python bit for bit; fmix32 is a
    bijection on sampled inputs with its published avalanche (each input bit
    flips about half the output bits); the kept fraction is within a binomial
    bound of (65536 - thr) / 65536; neighbouring columns, rows and seeds are
    uncorrelated; p = 0 keeps everything and p = 1 nothing.
    expert_forward / moe_forward / moe_backward take `keep` [N*k, F] (by
    assignment) and `scale`: h' = h * keep * scale feeds the down product.
add_rmsnorm / add_rmsnorm_np
    s = T(x + r); ss = sum s^2 in the router's lane/tree order; rstd =
    1 / sqrt(ss / d + eps); normed = T((s * rstd) * w) — fused_add_rmsnorm /
    RMSNorm (lib/blocks/_component.py:14, :17-20; eps 1e-6) in the order the C
    ABI fixes (g5moe_add_rmsnorm_router).  add_rmsnorm is C, add_rmsnorm_np an
    independent numpy restatement (bf16 rows, where s*s is exact in fp32).
    Pins: C == numpy bit for bit; C == exact-rational restatement on fp32 rows;
    power-of-two constant rows with eps = 0 give T(sign * w) exactly; the bf16
    add equals torch's bf16 add; within fp32 rounding of a float64 RMSNorm.
    Liger's own casting (LigerRMSNorm) stays unpinned: this is the contract's
    order, not Liger's.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None


def _clib():
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle.so"
        if not path.exists():
            from . import build as _b
            _b.build()
        L = ctypes.CDLL(str(path))
        P = ctypes.c_void_p
        L.g5o_router_logits_f32.argtypes = [P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P]
        L.g5o_router_logits_bf16.argtypes = [P, P, P, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                             P, P]
        L.g5o_topk.argtypes = [P, ctypes.c_int64, ctypes.c_int, ctypes.c_int, P, P]
        L.g5o_dispatch.argtypes = [P, ctypes.c_int64, ctypes.c_int, P, P, P, P]
        L.g5o_add_rmsnorm.argtypes = [P, P, ctypes.c_int, P, ctypes.c_float, ctypes.c_int64,
                                      ctypes.c_int, P, P, P]
        L.g5o_combine.argtypes = [P, P, P, P, ctypes.c_float, ctypes.c_int, ctypes.c_int64,
                                  ctypes.c_int, ctypes.c_int, P]
        L.g5o_input_grad.argtypes = [P, P, P, P, ctypes.c_int, ctypes.c_int64, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, P]
        for f in (L.g5o_router_logits_f32, L.g5o_router_logits_bf16, L.g5o_topk, L.g5o_dispatch,
                  L.g5o_add_rmsnorm, L.g5o_combine, L.g5o_input_grad):
            f.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _p(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(a: np.ndarray) -> np.ndarray:
    """Round to the nearest bf16 (ties to even), returned widened to fp32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u + (np.uint32(0x7FFF) + ((u >> 16) & 1))) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def widen(a: np.ndarray) -> np.ndarray:
    """uint16 bf16 bits -> fp32; float arrays pass through unchanged."""
    return bf16_to_f32(a) if a.dtype == np.uint16 else np.asarray(a)


# ---- router ------------------------------------------------------------------

def router_logits(x: np.ndarray, w: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    """C implementation.  x [N, d], w [E, d]: both fp32 or both uint16 bf16 bits."""
    N, d = x.shape
    E = w.shape[0]
    out = np.empty((N, E), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    if x.dtype == np.uint16:
        xx = np.ascontiguousarray(x)
        ww = np.ascontiguousarray(w, np.uint16)
        scratch = np.empty((E + 1) * d, dtype=np.float32)
        rc = _clib().g5o_router_logits_bf16(_p(xx), _p(ww), _p(b), N, d, E, _p(out), _p(scratch))
    else:
        xx = np.ascontiguousarray(x, np.float32)
        ww = np.ascontiguousarray(w, np.float32)
        rc = _clib().g5o_router_logits_f32(_p(xx), _p(ww), _p(b), N, d, E, _p(out))
    if rc != 0:
        raise ValueError("d must be a positive multiple of 64")
    return out


def router_logits_np(x_f32: np.ndarray, w_f32: np.ndarray, bias: Optional[np.ndarray] = None,
                     chunk: int = 4096) -> np.ndarray:
    """Vectorised numpy restatement of the same order.  Bit-exact with the C version
    when every product x*w is exact in fp32 (bf16 inputs); fp32 inputs need the
    fused multiply-add of the C version."""
    N, d = x_f32.shape
    E = w_f32.shape[0]
    L = d // 64
    W = np.ascontiguousarray(w_f32, np.float32).reshape(E, 64, L)
    out = np.empty((N, E), dtype=np.float32)
    for t0 in range(0, N, chunk):
        X = np.ascontiguousarray(x_f32[t0:t0 + chunk], np.float32).reshape(-1, 64, L)
        acc = np.zeros((X.shape[0], E, 64), dtype=np.float32)
        for i in range(L):
            acc = acc + X[:, None, :, i] * W[None, :, :, i]
        m = 32
        while m >= 1:
            acc = acc[..., :m] + acc[..., m:2 * m]
            m //= 2
        r = acc[..., 0]
        if bias is not None:
            r = r + np.asarray(bias, np.float32)[None, :]
        out[t0:t0 + chunk] = r
    return out


def topk_gates(logits: np.ndarray, k: int):
    """Scan top-k + renormalised softmax gates (numpy).  -> (idx int32 [N,k], w fp32 [N,k])."""
    N, E = logits.shape
    chosen = np.zeros((N, E), dtype=bool)
    idx = np.empty((N, k), dtype=np.int32)
    rows = np.arange(N)
    for s in range(k):
        best = np.full(N, -1, dtype=np.int64)
        bv = np.zeros(N, dtype=np.float32)
        for e in range(E):
            le = logits[:, e]
            take = (~chosen[:, e]) & ((best < 0) | (le > bv))
            best = np.where(take, e, best)
            bv = np.where(take, le, bv)
        idx[:, s] = best
        chosen[rows, best] = True
    l64 = logits.astype(np.float64)
    mx = l64.max(axis=1, keepdims=True)
    p = np.exp(l64 - mx)
    p /= p.sum(axis=1, keepdims=True)
    ps = np.take_along_axis(p, idx.astype(np.int64), axis=1)
    w = (ps / ps.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, w


def topk_gates_c(logits: np.ndarray, k: int):
    N, E = logits.shape
    lg = np.ascontiguousarray(logits, np.float32)
    idx = np.empty((N, k), dtype=np.int32)
    w = np.empty((N, k), dtype=np.float32)
    if _clib().g5o_topk(_p(lg), N, E, k, _p(idx), _p(w)) != 0:
        raise ValueError("bad k / E")
    return idx, w


# ---- dispatch ----------------------------------------------------------------

def dispatch(topk_idx: np.ndarray, n_experts: int):
    """-> counts [E], offsets [E+1], perm [N*k], inv_pos [N*k] (all int32)."""
    flat = np.ascontiguousarray(topk_idx, np.int64).reshape(-1)
    valid = (flat >= 0) & (flat < n_experts)
    key = np.where(valid, flat, n_experts)
    order = np.argsort(key, kind="stable")
    nvalid = int(valid.sum())
    perm = order[:nvalid].astype(np.int32)
    counts = np.bincount(flat[valid], minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    inv_pos = np.full(flat.shape[0], -1, dtype=np.int32)
    inv_pos[perm] = np.arange(nvalid, dtype=np.int32)
    return counts, offsets, perm, inv_pos


def dispatch_c(topk_idx: np.ndarray, n_experts: int):
    flat = np.ascontiguousarray(topk_idx, np.int32).reshape(-1)
    nk = flat.shape[0]
    counts = np.empty(n_experts, np.int32)
    offsets = np.empty(n_experts + 1, np.int32)
    perm = np.full(nk, -1, np.int32)
    inv_pos = np.empty(nk, np.int32)
    if _clib().g5o_dispatch(_p(flat), nk, n_experts, _p(counts), _p(offsets), _p(perm),
                            _p(inv_pos)) != 0:
        raise ValueError("n_experts > 64")
    return counts, offsets, perm[: int(offsets[-1])], inv_pos


# ---- experts and combine ---------------------------------------------------------

# ---- dropout mask (g5moe_dropout) -------------------------------------------------

_M32 = np.uint32(0xFFFFFFFF)


def _fmix32_np(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.uint32).copy()
    with np.errstate(over="ignore"):
        x ^= x >> np.uint32(16)
        x = (x.astype(np.uint64) * np.uint64(0x85EBCA6B) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        x ^= x >> np.uint32(13)
        x = (x.astype(np.uint64) * np.uint64(0xC2B2AE35) & np.uint64(0xFFFFFFFF)).astype(np.uint32)
        x ^= x >> np.uint32(16)
    return x


def dropout_threshold(p: float) -> int:
    """round(p * 65536), halves away from zero, of the fp32 value of p."""
    t = float(np.float32(p)) * 65536.0
    return min(65536, int(t + 0.5))


def dropout_scale(p: float) -> np.float32:
    """fp32 65536 / (65536 - thr); 0 when everything is dropped."""
    thr = dropout_threshold(p)
    return np.float32(0.0) if thr >= 65536 else np.float32(65536.0 / (65536 - thr))


def dropout_keep(assignments: np.ndarray, n_cols: int, p: float, seed: int) -> np.ndarray:
    """bool [len(assignments), n_cols]: the mask of each assignment's h row."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    lo, hi = np.uint32(seed & 0xFFFFFFFF), np.uint32(seed >> 32)
    a = np.asarray(assignments, dtype=np.int64).astype(np.uint32)
    key = _fmix32_np(((_fmix32_np(a ^ lo).astype(np.uint64) + np.uint64(hi))
                      & np.uint64(0xFFFFFFFF)).astype(np.uint32))
    pairs = np.arange((n_cols + 1) // 2, dtype=np.uint64)
    x = (key[:, None].astype(np.uint64) + pairs[None, :] * np.uint64(0x9E3779B9)) \
        & np.uint64(0xFFFFFFFF)
    bits = _fmix32_np(x.astype(np.uint32))
    r = np.empty((a.size, 2 * pairs.size), dtype=np.uint32)
    r[:, 0::2] = bits & np.uint32(0xFFFF)
    r[:, 1::2] = bits >> np.uint32(16)
    return r[:, :n_cols] >= np.uint32(dropout_threshold(p))


def _fmix32_py(x: int) -> int:
    x ^= x >> 16
    x = (x * 0x85EBCA6B) & 0xFFFFFFFF
    x ^= x >> 13
    x = (x * 0xC2B2AE35) & 0xFFFFFFFF
    x ^= x >> 16
    return x


def dropout_keep_py(a: int, f: int, p: float, seed: int) -> bool:
    """One mask element in plain Python integers (the pin of dropout_keep)."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    key = _fmix32_py((_fmix32_py((a & 0xFFFFFFFF) ^ (seed & 0xFFFFFFFF)) + (seed >> 32))
                     & 0xFFFFFFFF)
    bits = _fmix32_py((key + (f >> 1) * 0x9E3779B9) & 0xFFFFFFFF)
    r = (bits >> 16) if f & 1 else (bits & 0xFFFF)
    return r >= dropout_threshold(p)


def _silu(g: np.ndarray) -> np.ndarray:
    return g / (1.0 + np.exp(-g))


def expert_forward(x_f: np.ndarray, perm: np.ndarray, offsets: np.ndarray, top_k: int,
                   w_gate: np.ndarray, w_up: np.ndarray, w_down: np.ndarray,
                   dtype=np.float32, return_h: bool = False, storage: str = "fp32",
                   keep: Optional[np.ndarray] = None, scale: float = 1.0):
    """Per-expert SwiGLU over the routed rows, in `dtype` (float32 or float64).
    Weights may be uint16 bf16 bits or float arrays.  -> y_perm [N*k, d] (and h).

    storage="bf16" rounds h (the down product's input) and y_perm to bf16, the
    two points where the layer's bf16 dataflow stores bf16 — as the reference's
    bf16 FeedForward does with the SiLU-mul output and the `wo` output.
    keep (bool [N*k, F], indexed by assignment) and scale: dropout, h' = h * keep
    * scale before the rounding and the down product (h is then h')."""
    if storage not in ("fp32", "bf16"):
        raise ValueError(storage)
    E = w_gate.shape[0]
    F = w_gate.shape[1]
    d = x_f.shape[1]
    nk = perm.shape[0]
    y_perm = np.zeros((nk, d), dtype=dtype)
    h_all = np.zeros((nk, F), dtype=dtype) if return_h else None
    for e in range(E):
        o0, o1 = int(offsets[e]), int(offsets[e + 1])
        if o1 == o0:
            continue
        rows = x_f[perm[o0:o1] // top_k].astype(dtype, copy=False)
        wg = widen(w_gate[e]).astype(dtype, copy=False)
        wu = widen(w_up[e]).astype(dtype, copy=False)
        wd = widen(w_down[e]).astype(dtype, copy=False)
        h = _silu(rows @ wg.T) * (rows @ wu.T)
        if keep is not None:
            h = h * (keep[perm[o0:o1]].astype(dtype) * dtype(scale))
        if storage == "bf16":
            h = round_bf16(h).astype(dtype)
        y = h @ wd.T
        y_perm[o0:o1] = round_bf16(y) if storage == "bf16" else y
        if return_h:
            h_all[o0:o1] = h
    return (y_perm, h_all) if return_h else y_perm


def combine(y_perm: np.ndarray, inv_pos: np.ndarray, topk_w: np.ndarray) -> np.ndarray:
    N, k = topk_w.shape
    d = y_perm.shape[1]
    acc_t = np.float64 if y_perm.dtype == np.float64 else np.float32
    y = np.zeros((N, d), dtype=acc_t)
    ip = inv_pos.reshape(N, k)
    for s in range(k):
        p = ip[:, s]
        ok = p >= 0
        y[ok] = y[ok] + topk_w[ok, s:s + 1].astype(acc_t) * y_perm[p[ok]].astype(acc_t)
    return y


def moe_forward(x: np.ndarray, w_router: np.ndarray, w_gate: np.ndarray, w_up: np.ndarray,
                w_down: np.ndarray, top_k: int, bias: Optional[np.ndarray] = None,
                dtype=np.float32, return_h: bool = False, storage: str = "fp32",
                dropout: Optional[tuple] = None) -> dict:
    """Whole layer.  x / w_router: fp32 or uint16 bf16 bits (same kind).  Expert
    weights: bf16 bits or float arrays.  dropout = (p, seed): the mask of
    dropout_keep on h.  Returns every intermediate."""
    E = w_router.shape[0]
    logits = router_logits(x, w_router, bias)
    idx, w = topk_gates_c(logits, top_k)
    counts, offsets, perm, inv_pos = dispatch_c(idx, E)
    xf = widen(x)
    if storage == "bf16" and x.dtype != np.uint16:
        xf = round_bf16(xf)  # an fp32 x enters the bf16 expert GEMMs rounded to bf16
    keep, scale = None, 1.0
    if dropout is not None and dropout[0] > 0:
        keep = dropout_keep(np.arange(perm.size), w_gate.shape[1], dropout[0], dropout[1])
        scale = float(dropout_scale(dropout[0]))
    res = expert_forward(xf, perm, offsets, top_k, w_gate, w_up, w_down, dtype=dtype,
                         return_h=return_h, storage=storage, keep=keep, scale=scale)
    y_perm, h = res if return_h else (res, None)
    y = combine(y_perm, inv_pos, w)
    out = dict(logits=logits, topk_idx=idx, topk_w=w, counts=counts, offsets=offsets,
               perm=perm, inv_pos=inv_pos, y_perm=y_perm, y=y)
    if return_h:
        out["h"] = h
    return out


# ---- pre-norm (residual add + RMSNorm) and combine in the C ABI's order ------------

def _rows(a: np.ndarray):
    """-> (contiguous array, dtype code 0 = bf16 bits, 1 = fp32)."""
    if a.dtype == np.uint16:
        return np.ascontiguousarray(a), 0
    return np.ascontiguousarray(a, np.float32), 1


def add_rmsnorm(residual: np.ndarray, weight: np.ndarray, eps: float,
                x_add: Optional[np.ndarray] = None):
    """C implementation.  Rows as uint16 bf16 bits or fp32 (x_add of the same kind).
    -> (normed, sum) in the input's representation; sum is None without x_add."""
    r, code = _rows(residual)
    N, d = r.shape
    xa = None
    if x_add is not None:
        xa, c2 = _rows(x_add)
        if c2 != code or xa.shape != r.shape:
            raise ValueError("x_add must match residual")
    w = np.ascontiguousarray(weight, np.float32)
    normed = np.empty_like(r)
    ssum = np.empty_like(r) if xa is not None else None
    scratch = np.empty(d, np.float32)
    if _clib().g5o_add_rmsnorm(_p(xa), _p(r), code, _p(w), float(eps), N, d, _p(ssum),
                               _p(normed), _p(scratch)) != 0:
        raise ValueError("d must be a positive multiple of 64")
    return normed, ssum


def add_rmsnorm_np(residual_f32: np.ndarray, weight: np.ndarray, eps: float,
                   x_add_f32: Optional[np.ndarray] = None):
    """Vectorised numpy restatement for bf16 rows (given widened to fp32): every
    s * s is exact in fp32, so the lane fma chain is a chain of fp32 adds.
    -> (normed, sum) as fp32 arrays holding bf16 values."""
    s = np.asarray(residual_f32, np.float32)
    if x_add_f32 is not None:
        s = round_bf16(np.asarray(x_add_f32, np.float32) + s)
    N, d = s.shape
    L = d // 64
    S = s.reshape(N, 64, L)
    acc = np.zeros((N, 64), np.float32)
    for i in range(L):
        acc = acc + S[:, :, i] * S[:, :, i]
    m = 32
    while m >= 1:
        acc = acc[:, :m] + acc[:, m:2 * m]
        m //= 2
    ss = acc[:, 0]
    rstd = np.float32(1.0) / np.sqrt(ss / np.float32(d) + np.float32(eps))
    normed = round_bf16((s * rstd[:, None]) * np.asarray(weight, np.float32)[None, :])
    return normed, (s if x_add_f32 is not None else None)


def input_grad_c(dxp_bits: np.ndarray, inv_pos: np.ndarray, dlogits: np.ndarray,
                 w_router: np.ndarray, out_dtype: str = "bf16") -> np.ndarray:
    """C restatement of g5moe_input_grad: per column, the dX_perm rows added in slot
    order from 0 (rows with a negative position skipped), then fmaf of dlogits and
    the router weight in expert order, one rounding to out_dtype.  dxp as uint16
    bf16 bits [N*k, d]; w_router and the result as uint16 bits ("bf16") or fp32."""
    dl = np.ascontiguousarray(dlogits, np.float32)
    N, E = dl.shape
    ip = np.ascontiguousarray(inv_pos, np.int32).reshape(N, -1)
    k = ip.shape[1]
    xp = np.ascontiguousarray(dxp_bits, np.uint16)
    d = xp.shape[1]
    code = 0 if out_dtype == "bf16" else 1
    wr = np.ascontiguousarray(w_router, np.uint16 if code == 0 else np.float32)
    out = np.empty((N, d), np.uint16 if code == 0 else np.float32)
    if _clib().g5o_input_grad(_p(xp), _p(ip), _p(dl), _p(wr), code, N, d, k, E, _p(out)) != 0:
        raise ValueError("bad dtype")
    return out


def combine_c(y_perm_bits: np.ndarray, inv_pos: np.ndarray, topk_w: np.ndarray,
              residual: Optional[np.ndarray] = None, alpha: float = 1.0,
              out_dtype: str = "bf16") -> np.ndarray:
    """C restatement of g5moe_combine (residual None) / g5moe_combine_residual.
    y_perm as uint16 bf16 bits; residual and the result in out_dtype's
    representation (uint16 bits for "bf16", fp32 for "f32")."""
    N, k = topk_w.shape
    yp = np.ascontiguousarray(y_perm_bits, np.uint16)
    d = yp.shape[1]
    code = 0 if out_dtype == "bf16" else 1
    out = np.empty((N, d), np.uint16 if code == 0 else np.float32)
    r = None
    if residual is not None:
        r, c2 = _rows(residual)
        if c2 != code:
            raise ValueError("residual dtype must match out_dtype")
    ip = np.ascontiguousarray(inv_pos, np.int32).reshape(-1)
    w = np.ascontiguousarray(topk_w, np.float32)
    if _clib().g5o_combine(_p(yp), _p(ip), _p(w), _p(r), float(alpha), code, N, d, k,
                           _p(out)) != 0:
        raise ValueError("bad dtype")
    return out


# ---- backward ----------------------------------------------------------------------

def moe_backward(x: np.ndarray, w_router: np.ndarray, w_gate: np.ndarray, w_up: np.ndarray,
                 w_down: np.ndarray, topk_idx: np.ndarray, dy: np.ndarray,
                 grad_logits: Optional[np.ndarray] = None,
                 bias: Optional[np.ndarray] = None,
                 keep: Optional[np.ndarray] = None, scale: float = 1.0) -> dict:
    """Textbook float64 backward of the layer for the routing indices topk_idx
    (the top-k choice is piecewise constant in the logits, so it carries no
    gradient).  Forward: logits = x Wr^T (+ b); w = softmax over the chosen
    logits; per assignment (t, s) with e = topk_idx[t, s]:
    h = silu(x Wg_e^T) * (x Wu_e^T), Y = h Wd_e^T; y[t] = sum_s w[t, s] Y[t, s]
    (FeedForward.forward, lib/blocks/_component.py:48-52, per expert).  The loss
    is L(y, logits) with dL/dy = dy and an optional dL/dlogits = grad_logits.
    Inputs: float arrays or uint16 bf16 bits (widened).  keep (bool [N*k, F], by
    assignment t*k + s) and scale: dropout on h, h' = h * keep * scale feeds the
    down product, so dWd uses h' and the SwiGLU derivative takes dh' * keep *
    scale.  Returns dict with dx, d_w_router, d_w_gate, d_w_up, d_w_down,
    dlogits, dw, y."""
    f = lambda a: widen(a).astype(np.float64)
    X, Wr, Wg, Wu, Wd, DY = f(x), f(w_router), f(w_gate), f(w_up), f(w_down), f(dy)
    N, d = X.shape
    E, F = Wg.shape[0], Wg.shape[1]
    idx = np.asarray(topk_idx, np.int64)
    k = idx.shape[1]
    logits = X @ Wr.T
    if bias is not None:
        logits = logits + np.asarray(bias, np.float64)[None, :]
    ls = np.take_along_axis(logits, idx, axis=1)
    ls = ls - ls.max(axis=1, keepdims=True)
    w = np.exp(ls) / np.exp(ls).sum(axis=1, keepdims=True)
    dx = np.zeros_like(X)
    dwg, dwu, dwd = np.zeros_like(Wg), np.zeros_like(Wu), np.zeros_like(Wd)
    dw = np.zeros((N, k))
    y = np.zeros_like(X)
    for s in range(k):
        for e in range(E):
            rows = np.nonzero(idx[:, s] == e)[0]
            if rows.size == 0:
                continue
            xe = X[rows]
            g, u = xe @ Wg[e].T, xe @ Wu[e].T
            sg = 1.0 / (1.0 + np.exp(-g))
            h = g * sg * u
            m = 1.0
            if keep is not None:
                m = keep[rows * k + s].astype(np.float64) * float(scale)
                h = h * m
            Y = h @ Wd[e].T
            we = w[rows, s:s + 1]
            y[rows] += we * Y
            dw[rows, s] = (DY[rows] * Y).sum(axis=1)
            dY = we * DY[rows]
            dwd[e] += dY.T @ h
            dh = (dY @ Wd[e]) * m
            dg = dh * u * sg * (1.0 + g * (1.0 - sg))
            du = dh * g * sg
            dwg[e] += dg.T @ xe
            dwu[e] += du.T @ xe
            dx[rows] += dg @ Wg[e] + du @ Wu[e]
    dl_sel = w * (dw - (w * dw).sum(axis=1, keepdims=True))
    dlogits = np.zeros((N, E))
    np.put_along_axis(dlogits, idx, dl_sel, axis=1)
    if grad_logits is not None:
        dlogits = dlogits + np.asarray(grad_logits, np.float64)
    dx += dlogits @ Wr
    return dict(dx=dx, d_w_router=dlogits.T @ X, d_w_gate=dwg, d_w_up=dwu, d_w_down=dwd,
                dlogits=dlogits, dw=dw, y=y)
