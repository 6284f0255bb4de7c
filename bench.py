"""Benchmark: GeneT5 MoE layer forward (16 experts, top-2, SwiGLU d=768 F=3072) on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config 2|3] [--no-cpu-baseline]

A step is one whole layer forward (router + dispatch in one g5moe_route call ->
gate|up GEMM + SwiGLU -> down GEMM -> combine) through the C ABI's stage entry points, on synthetic
inputs already resident in HBM (config 2: 36,400 tokens bf16, uniform routing).
Prints ONE JSON line.  `value` is tokens/s of the whole layer; `roofline` is
for the dominant kernel (the grouped gate|up GEMM), its average launch time
taken from HIP events recorded around it, on the stream it runs on, inside the
timed loop (which records events only around the two expert GEMMs, created
without a system-scope fence so that recording them costs the stream nothing;
`stage_ms` holds every stage's time from a second loop of the same steps with
an event at each stage boundary).  `cpu_baseline` times the CPU oracle (fp32,
numpy/BLAS) on the same workload (all of its tokens unless --cpu-sample-tokens
bounds it) on this host's cores, and config 1 beside it; `torch_eager_gpu` times
the same layer written as eager PyTorch on the same GPU (the reference's
FeedForward body per expert), for context.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "MoE layer tokens/s + expert-GEMM TFLOP/s (% bf16 peak), 36.4k tok, 16e top-2"
PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4, 5))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--train", action="store_true",
                    help="time the training step instead: MoEFeedForward's forward and its "
                         "autograd backward, with a per-stage breakdown")
    ap.add_argument("--dropout", type=float, default=0.1,
                    help="--train: dropout on the expert hidden state (GeneT5 trains with 0.1)")
    ap.add_argument("--cpu-sample-tokens", type=int, default=0,
                    help="tokens of the workload the CPU baseline runs (0: all of them)")
    ap.add_argument("--shard", choices=("dp8", "ep8"), default=None,
                    help="one GPU's share of config 2 sharded over 8 GPUs: dp8 = 4,550 tokens "
                         "with all 16 experts (about 569 rows per expert), ep8 = the 2 experts "
                         "one GPU owns with their 4,550 rows each (4,550 tokens routed top-2 of "
                         "2); the layer's kernels at those shapes, no exchange")
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="untimed calls of the step for this many milliseconds of wall time "
                         "before the warm-up steps (0: none): after an idle spell the "
                         "board's power controller lets the clock overshoot, then holds it "
                         "low for about 20 ms before it settles, and the timed steps should "
                         "see the steady state a continuously running layer sees")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after the benchmark, run a 256 MiB elementwise copy (read 256 MiB, "
                         "write 256 MiB) whose FETCH_SIZE / WRITE_SIZE counters scale the "
                         "GEMM's counters to bytes")
    return ap.parse_args()


def cpu_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"]
        return int(max(n)) if n else 1
    except Exception:
        return 1


def cpu_baseline(inp, n_sample: int) -> dict:
    """Oracle (fp32 numpy/BLAS) on the first n_sample tokens of the workload (all of
    them by default: config 2 takes about 1.3 s per run on a 16-thread host)."""
    import oracle
    from genet5_amd import synth
    x = inp.x[:n_sample]
    wg = synth.bf16_bits_to_f32(inp.w_gate)
    wu = synth.bf16_bits_to_f32(inp.w_up)
    wd = synth.bf16_bits_to_f32(inp.w_down)
    run = lambda: oracle.moe_forward(x, inp.w_router, wg, wu, wd, inp.top_k, bias=inp.bias)
    run()  # warm-up
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    return {
        "value": n_sample / t,
        "unit": "tokens/s",
        "cores": blas_threads(),
        "kind": "port",
        "sample": (f"oracle.moe_forward (C router + numpy fp32 BLAS experts) on "
                   + ("all " if n_sample == inp.x.shape[0] else "the first ")
                   + f"{n_sample} tokens of the same workload, median of 3 after 1 warm-up, "
                   f"{t * 1e3:.1f} ms per run; host {cpu_info()}, os.cpu_count()={os.cpu_count()}"),
        "expert_tflops": 6 * 768 * 3072 * n_sample * inp.top_k / t / 1e12,
    }


def eager_layer(x, wr, bias, w_gate, w_up, w_down, k, dropout=0.0):
    """The layer as PyTorch code would write it: the reference's FeedForward
    (lib/blocks/_component.py:48-52: silu(wi_0(x)) * wi_1(x), dropout on that
    product in training, then wo) per expert over its routed rows, an fp32 router
    with torch.softmax / torch.topk, and an index_add combine.  bf16 weights and
    activations through F.linear (hipBLASLt); the per-expert row lists cost a host
    synchronisation each (nonzero), as in any such loop."""
    import torch
    import torch.nn.functional as Fn
    logits = x.float() @ wr.float().t()
    if bias is not None:
        logits = logits + bias
    wts, idx = torch.topk(torch.softmax(logits, dim=-1), k, dim=-1)
    wts = wts / wts.sum(-1, keepdim=True)
    y = torch.zeros(x.shape, dtype=torch.float32, device=x.device)
    for e in range(w_gate.shape[0]):
        tok, slot = (idx == e).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        xe = x[tok]
        h = Fn.silu(Fn.linear(xe, w_gate[e])) * Fn.linear(xe, w_up[e])
        if dropout > 0.0:
            h = Fn.dropout(h, dropout, training=True)
        y = y.index_add(0, tok, Fn.linear(h, w_down[e]).float() * wts[tok, slot, None])
    return y.to(x.dtype)


def torch_eager_gpu(x, wr, bias, w_gate, w_up, w_down, k, ref_y, steps=10, warmup=3) -> dict:
    """eager_layer on the same GPU and tensors, beside the HIP layer, with the
    difference between the two outputs."""
    import torch

    def fwd():
        return eager_layer(x, wr, bias, w_gate, w_up, w_down, k)

    for _ in range(warmup):
        out = fwd()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = fwd()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    err = (out.float() - ref_y.float()).abs()
    ref_abs = ref_y.float().abs()
    return {"ms_per_step": ms, "tokens_per_s": x.shape[0] / (ms * 1e-3),
            # a token whose top-2 is a near tie may pick another expert in fp32
            # torch than in the fixed-order router: the mean is the comparison
            "mean_rel_diff_vs_hip": err.mean().item() / max(ref_abs.mean().item(), 1e-30),
            "max_rel_diff_vs_hip": err.max().item() / max(ref_abs.max().item(), 1e-30),
            "what": "PyTorch eager on this GPU: fp32 router + softmax/topk, per-expert "
                    "F.linear SwiGLU MLP over the routed rows (bf16, hipBLASLt), index_add "
                    f"combine; {steps} steps after {warmup} warm-up"}


def torch_eager_gpu_train(x, wr, w_gate, w_up, w_down, k, dy, dropout, steps=5,
                          warmup=2) -> dict:
    """eager_layer's forward and autograd backward (parameter and input gradients)
    on the same GPU, as PyTorch training code would run the layer."""
    import torch
    params = [t.detach().clone().requires_grad_(True) for t in (wr, w_gate, w_up, w_down)]
    xr = x.detach().clone().requires_grad_(True)

    def step():
        for t in params + [xr]:
            t.grad = None
        y = eager_layer(xr, params[0], None, params[1], params[2], params[3], k, dropout)
        y.backward(dy)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"ms_per_step": ms, "tokens_per_s": x.shape[0] / (ms * 1e-3),
            "what": "PyTorch eager forward + autograd backward of the same layer on this "
                    f"GPU (bf16 parameters, dropout {dropout}); {steps} steps after "
                    f"{warmup} warm-up"}


SETTLE_WHY = ("untimed calls of the step before the warm-up steps: after an idle spell the "
              "board's power controller first lets the shader clock run high, then holds it "
              "low for about 20 ms before it settles (gate|up 604 -> 874 -> 607 us per call "
              "over the first 25 ms in profiles/moe_layer_cfg2_kernel_stats.md), so without "
              "them a short timed region measures that transient instead of the steady state")


class TimingEvent:
    """A HIP event used only for timing, created with hipEventDisableSystemFence.

    torch.cuda.Event(enable_timing=True) is a default HIP event: recording it
    performs a system-scope release (the L2 written back and invalidated), which
    leaves a gap of several microseconds before the next kernel on the stream
    and a cold L2 behind it.  An event created with hipEventDisableSystemFence
    still timestamps its place in the stream, and hipEventElapsedTime still reads
    it once the device has been synchronised.  The event comes from the HIP
    runtime torch has loaded (RTLD_NOLOAD), so it shares torch's streams.
    """

    DISABLE_SYSTEM_FENCE = 0x20000000   # hipEventDisableSystemFence (hip_runtime_api.h)
    _hip = None

    def __init__(self):
        import ctypes
        if TimingEvent._hip is None:
            TimingEvent._hip = ctypes.CDLL("libamdhip64.so.7",
                                           mode=os.RTLD_NOLOAD | ctypes.RTLD_GLOBAL)
        self._c = ctypes
        self.h = ctypes.c_void_p()
        rc = self._hip.hipEventCreateWithFlags(ctypes.byref(self.h),
                                               ctypes.c_uint(self.DISABLE_SYSTEM_FENCE))
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream) -> None:
        rc = self._hip.hipEventRecord(self.h, self._c.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end: "TimingEvent") -> float:
        ms = self._c.c_float()
        rc = self._hip.hipEventElapsedTime(self._c.byref(ms), self.h, end.h)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if self._hip is not None and self.h:
            self._hip.hipEventDestroy(self.h)


def settle(fn, ms: float) -> dict:
    """Call fn (untimed) for `ms` milliseconds of wall time, in groups of four calls
    with a device synchronisation after each group; returns the settle record of the
    JSON line."""
    import torch
    n = 0
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            fn()
        n += 4
        torch.cuda.synchronize()
    return {"ms": round((time.perf_counter() - t0) * 1e3, 1), "calls": n, "why": SETTLE_WHY}


def timed(fn, steps: int, warmup: int, settle_ms: float = 0.0) -> float:
    import torch
    settle(fn, settle_ms)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def bench_config4(args) -> dict:
    """12 stacked RMSNorm -> MoE -> residual blocks on 45,500 packed tokens (config 4)."""
    import torch
    from genet5_amd.harness import blocks
    dev = torch.device("cuda:0")
    cfg = blocks.make_config4()
    stack = blocks.MoEStack(12, 768, 3072).to(dev).to(torch.bfloat16)
    blocks.load_layer_weights(stack, cfg.layer_seeds, 3072)
    x = torch.from_numpy(cfg.x).view(torch.bfloat16).to(dev)
    N = x.shape[1]
    with torch.no_grad():
        t = timed(lambda: stack(x), args.steps, args.warmup, args.settle_ms)
        # the same stack as the torch composition RMSNorm -> MoE -> residual add
        stack.set_fused(False)
        t_unfused = timed(lambda: stack(x), args.steps, args.warmup, args.settle_ms)
        stack.set_fused(True)
    flops = 12 * 6 * 768 * 3072 * N * 2
    # the two fused memory-bound entry points on this batch (HIP events, 20 calls each)
    from genet5_amd import _lib, ops
    layer = stack.layers[0]
    x2 = x.reshape(-1, 768)
    nw = layer.norm.weight.float().contiguous()
    wr = layer.ff.router.weight.contiguous()
    xa = torch.randn_like(x2)
    with torch.no_grad():
        normed, _, idx, w = ops.add_rmsnorm_router(x2, nw, 1e-6, wr, 2)
        _, offsets, perm, inv_pos = ops.dispatch(idx, 16, 768)
        wgu, wd = layer.ff._expert_weights()
        y_perm = ops.expert_swiglu(normed, perm, offsets, wgu, wd, 2)

    def ev_time(fn, reps=20):
        fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e-3
    t_norm = ev_time(lambda: ops.add_rmsnorm_router(x2, nw, 1e-6, wr, 2))
    t_addnorm = ev_time(lambda: ops.add_rmsnorm_router(x2, nw, 1e-6, wr, 2, x_add=xa))
    t_comb = ev_time(lambda: ops.combine_residual(y_perm, inv_pos, w, x2, 1.0))
    ws4 = ops.workspace(_lib.make_shape(N, 768, 3072, 16, 2, _lib.DTYPE_BF16), dev)
    t_route = ev_time(lambda: ops.add_rmsnorm_route(x2, nw, 1e-6, wr, 2, x_add=xa, ws=ws4,
                                                    d_ff=3072))
    t_unroute = ev_time(lambda: ops.dispatch(
        ops.add_rmsnorm_router(x2, nw, 1e-6, wr, 2, x_add=xa)[2], 16, 768))
    nd2 = N * 768 * 2
    kernels = {
        "rmsnorm_router_us": t_norm * 1e6,
        "rmsnorm_router_gbs": (2 * nd2 + N * 16) / t_norm / 1e9,
        "add_rmsnorm_router_us": t_addnorm * 1e6,
        "add_rmsnorm_router_gbs": (4 * nd2 + N * 16) / t_addnorm / 1e9,
        "combine_residual_us": t_comb * 1e6,
        "add_rmsnorm_route_us": t_route * 1e6,
        "add_rmsnorm_router_then_dispatch_us": t_unroute * 1e6,
        "combine_residual_gbs": (2 * nd2 + N * 2 * 768 * 2 + N * 16) / t_comb / 1e9,
        "bytes": "rmsnorm_router: read rows, write normed, write idx/w (8 B/token each); "
                 "add_: + read x_add, write the sum; combine_residual: read y_perm (k rows), "
                 "residual, write out, read inv_pos/w; add_rmsnorm_route: add_rmsnorm_router "
                 "with the dispatch (two launches), against the two calls in three",
    }
    return {
        "metric": "12-block RMSNorm->MoE->residual stack tokens/s, 45.5k packed tok, 16e top-2",
        "value": N / t, "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle": {"ms_per_loop": args.settle_ms, "why": SETTLE_WHY},
        "ms_per_step": t * 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "cfg4: 12 x (RMSNorm, MoE, residual), 45,500 tokens packed from "
                               "lengths U[1000, 9000], seeded N(0, 0.02) weights per layer",
                   "n_tokens": N, "n_layers": 12, "n_sequences": len(cfg.cu_seqlens) - 1},
        "expert_gemm_tflops_incl_layer_overheads": flops / t / 1e12,
        "blocks": "fused: g5moe_add_rmsnorm_route + experts + g5moe_combine_residual",
        "unfused_ms_per_step": t_unfused * 1e3,
        "fused_kernels": kernels,
    }


def bench_config5(args) -> dict:
    """Encoder (ALiBi torch attention + HIP MoE) driven by 16-step MDLM unmasking (config 5)."""
    import torch
    from genet5_amd.harness import encoder
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = encoder.GeneT5MoE().to(dev)
    with torch.no_grad():
        for p in model.parameters():
            if p.dim() >= 2:
                p.normal_(0, 0.02)
    model = model.to(torch.bfloat16).eval()
    g = torch.Generator(device="cpu").manual_seed(0)
    mask_id, pad_id = 4095, 0
    prefix = torch.randint(1, 4095, (8, 2275), generator=g).to(dev)
    stats = {}
    run = lambda: encoder.diffusion_generate(model, prefix, 2275, mask_id, pad_id, num_steps=16,
                                             stats=stats)
    # the same run with attention in the PyTorch reference composition (SDPA with
    # the ALiBi bias as a mask), as BASELINE's config 5 states it
    model.set_attention_backend("torch")
    with torch.no_grad():
        model(torch.cat([prefix, prefix], 1))  # warm-up forward
    t_torch_attn = timed(run, 1, 0)
    model.set_attention_backend("hip")
    with torch.no_grad():
        model(torch.cat([prefix, prefix], 1))  # warm-up forward
    t = timed(run, 1, 0)
    fw = stats["forwards"]
    n_tok = 8 * 4550
    # the attention kernel alone at this shape, on the model's own layer-0 inputs
    from genet5_amd import attention as attn_mod
    layer0 = model.layers[0]
    with torch.no_grad():
        h = model.embed(torch.cat([prefix, prefix], 1))
        hn = layer0.norm1(h)
        q = layer0.self_attn.q(hn).view(-1, 12, 64)
        k = layer0.self_attn.k(hn).view(-1, 12, 64)
        v = layer0.self_attn.v(hn).view(-1, 12, 64)
    cu = torch.arange(0, 9 * 4550, 4550, dtype=torch.int32, device=dev)
    sl = layer0.self_attn.slopes_on(dev)
    att = {}
    for name, skip in (("skip", True), ("dense", False)):
        f = lambda: attn_mod.attn_varlen_fwd(q, k, v, cu, 4550, 0.125, sl, key_bounds=skip)
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            f()
        e1.record()
        torch.cuda.synchronize()
        att[name] = e0.elapsed_time(e1) / 20
    attn_flop = 4.0 * 8 * 4550 * 4550 * 64 * 12
    return {
        "metric": "MDLM 16-step unmasking, encoder tokens/s (12 layers, HIP ALiBi attention + HIP MoE)",
        "value": n_tok * fw / t, "unit": "tokens/s", "n_gpus": 1, "steps": 1, "warmup": 1,
        "ms_per_step": t * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "cfg5: 8 x 4,550 tokens (2,275 prefix + 2,275 [MASK]), vocab 4,096, "
                               "12 layers, 16 unmasking steps + final fill, argmax",
                   "attention": "HIP varlen ALiBi kernel (torch SDPA composition timed beside it)",
                   "forwards": fw, "n_tokens_per_forward": n_tok},
        "moe_expert_tflop_total": 12 * fw * 6 * 768 * 3072 * n_tok * 2 / 1e12,
        "torch_attention_ms_per_step": t_torch_attn * 1e3,
        "torch_attention_tokens_per_s": n_tok * fw / t_torch_attn,
        "attention_kernel": {
            "shape": "8 x 4,550 tokens, 12 heads, head_dim 64, ALiBi, layer-0 inputs",
            "ms_skip": att["skip"], "ms_dense": att["dense"],
            "dense_equivalent_tflops_skip": attn_flop / att["skip"] / 1e9,
            "tflops_dense": attn_flop / att["dense"] / 1e9},
    }


def train_stage_breakdown(args) -> dict:
    """The module's training step as its stages, for the per-stage times: the forward
    (router with logits and the dispatch, experts keeping the gate|up products, combine) and
    every backward stage (gate/router gradients, the dh GEMM with the SwiGLU
    backward in its epilogue, dX GEMM, input gradient, weight-gradient operands, the
    expert weight gradients from the forward's h, the router weight gradient) through
    the C ABI — the kernels
    ops.moe_backward enqueues for the module — with one HIP event between
    consecutive stages on the stream they run on (no dropout)."""
    import ctypes
    import torch
    from genet5_amd import _lib, ops, synth
    dev = torch.device("cuda:0")
    inp = synth.make_config(args.config, seed=0)
    N, d = inp.x.shape
    E, F = inp.w_gate.shape[0], inp.w_gate.shape[1]
    k = inp.top_k
    tt = synth.to_torch(inp, dev)
    x, wr = tt["x"], tt["w_router"]
    wgu = ops.pack_gate_up(tt["w_gate"], tt["w_up"])
    wd = tt["w_down"]
    wd_t, wgu_t = ops.transpose_experts(wd), ops.transpose_experts(wgu)
    dy = (torch.randn(N, d, device=dev) * 0.01).to(torch.bfloat16)
    shape = _lib.make_shape(N, d, F, E, k, _lib.DTYPE_BF16)
    P, S = ops._ptr, ops._stream(dev)
    stream = torch.cuda.current_stream(dev)
    names = ["fwd", "gate_router_grad", "dh_swiglu", "dx_gemm", "input_grad",
             "wgrad_operands", "wgrad_gemms", "router_wgrad"]

    # the expert offsets reach the host by a non-blocking copy issued right after
    # the forward's dispatch, so reading them does not drain the queue
    offs_host = torch.empty(E + 1, dtype=torch.int32, pin_memory=True)
    offs_ready = torch.cuda.Event()

    def step(ev=None):
        rec = (lambda i: ev[i].record(stream)) if ev is not None else (lambda i: None)
        rec(0)
        y, logits, idx, w, offsets, perm, inv_pos, y_perm, fac, h = ops.moe_forward_train(
            x, wr, wgu, wd, k, offsets_host=offs_host, offsets_ready=offs_ready, return_h=True,
            factors=True)
        rec(1)
        offs_ready.synchronize()
        offs = offs_host.tolist()
        kmax = ops.wgrad_kmax(max(b - a for a, b in zip(offs[:-1], offs[1:])))
        dw = torch.empty((N, k), dtype=torch.float32, device=dev)
        dy_buf = torch.empty((E * kmax + ops.ROW_PAD, d), dtype=torch.bfloat16, device=dev)
        _lib.call("g5moe_gate_grad_padded", P(dy), P(y_perm), P(inv_pos), P(w), P(offsets),
                  P(dw), P(dy_buf), kmax, ctypes.byref(shape), S)
        dl = torch.empty((N, E), dtype=torch.float32, device=dev)
        _lib.call("g5moe_router_grad", P(dw), P(w), P(idx), None, P(dl), ctypes.byref(shape), S)
        rec(2)
        dgu_buf = torch.empty((E * kmax + ops.ROW_PAD, 2 * F), dtype=torch.bfloat16, device=dev)
        dgu_pad = dgu_buf[:E * kmax].view(E, kmax, 2 * F)
        _lib.call("g5moe_dh_swiglu_backward", P(dy_buf), kmax, P(offsets), P(wd_t), P(fac),
                  P(dgu_buf), ctypes.byref(shape), S)
        rec(3)
        dxp = ops.grouped_gemm_padded(dgu_buf, kmax, N * k, offsets, wgu_t)
        rec(4)
        dx = torch.empty((N, d), dtype=torch.bfloat16, device=dev)
        _lib.call("g5moe_input_grad", P(dxp), P(inv_pos), P(dl), P(wr), P(dx),
                  ctypes.byref(shape), S)
        rec(5)
        dy_pad = dy_buf[:E * kmax].view(E, kmax, d)
        x_pad = ops.pad_rows(x, perm, offsets, E, kmax, k)
        rec(6)
        d_wd = torch.empty((E, d, F), dtype=torch.bfloat16, device=dev)
        d_wg = torch.empty((E, F, d), dtype=torch.bfloat16, device=dev)
        d_wu = torch.empty((E, F, d), dtype=torch.bfloat16, device=dev)
        _lib.call("g5moe_weight_grad_sorted_h", P(dy_pad), P(h), P(d_wd), P(dgu_pad), P(x_pad),
                  P(d_wg), P(d_wu), P(offsets), kmax, ctypes.byref(shape), S)
        rec(7)
        ops.router_weight_grad(dl, x, shape)
        rec(8)

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
              for _ in range(args.steps)]
    settled = settle(step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    st = {n: sum(ev[j].elapsed_time(ev[j + 1]) for ev in events) / args.steps
          for j, n in enumerate(names)}
    g = 2 * d * F * N * k  # one d x F product over the routed rows
    flops = {"dh_swiglu": g, "dx_gemm": 2 * g, "wgrad_gemms": 3 * g}
    return {"stage_ms": st, "stage_ms_per_step": ms,
            "stage_tflops": {n: flops[n] / (st[n] * 1e-3) / 1e12 for n in flops}}


def bench_train(args) -> dict:
    """Training step of the layer at config 2 as GeneT5 runs it: y = module(x) then
    y.backward(dy) through autograd, with MoEFeedForward(768, 3072, dropout) in train
    mode (bf16 parameters, as GeneT5 holds the model) and x requiring grad.  Before
    every step the module's cache of packed and transposed expert weights is
    dropped, as an optimizer step changing the weights would, so they are rebuilt
    each step (the optimizer's own kernels are not timed);
    `accumulation_ms_per_step` is the same step with them cached (micro-steps of
    gradient accumulation).  Dropout defaults to GeneT5's 0.1
    (`dropout_zero_ms_per_step` without it).  The per-stage breakdown comes from the
    same kernels enqueued stage by stage (train_stage_breakdown)."""
    import torch
    from genet5_amd import synth
    from genet5_amd import moe as moe_mod
    from genet5_amd.moe import MoEFeedForward
    dev = torch.device("cuda:0")
    inp = synth.make_config(args.config, seed=0)
    N, d = inp.x.shape
    E, F = inp.w_gate.shape[0], inp.w_gate.shape[1]
    k = inp.top_k
    tt = synth.to_torch(inp, dev)
    x = tt["x"]
    m = MoEFeedForward(d, F, args.dropout, num_experts=E, top_k=k).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        m.router.weight.copy_(tt["w_router"])
        m.w_gate.copy_(tt["w_gate"])
        m.w_up.copy_(tt["w_up"])
        m.w_down.copy_(tt["w_down"])
    m.train()
    dy = (torch.randn(N, d, device=dev) * 0.01).to(torch.bfloat16)
    xr = x.clone().requires_grad_(True)

    def step(update=True):
        if update:
            # what an optimizer step does to the layer's caches (its own kernels are
            # not the layer's): the packed and transposed weights are rebuilt
            moe_mod.clear_weight_cache()
        m.zero_grad(set_to_none=True)
        xr.grad = None
        y = m(xr)
        y.backward(dy)

    def run(steps, warmup, update):
        settle(lambda: step(update), args.settle_ms)
        for _ in range(warmup):
            step(update)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step(update)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    ms = run(args.steps, args.warmup, True)
    ms_acc = run(args.steps, 2, False)
    p_saved = m.dropout
    m.dropout = 0.0
    ms_p0 = run(args.steps, 2, True)
    m.dropout = p_saved
    bd = train_stage_breakdown(args)
    eager = torch_eager_gpu_train(x, tt["w_router"], tt["w_gate"], tt["w_up"], tt["w_down"], k,
                                  dy, args.dropout)
    g = 2 * d * F * N * k
    return {
        "metric": "MoE layer training step (forward + backward) tokens/s, 36.4k tok, 16e top-2",
        "value": N / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "settle": {"ms_per_loop": args.settle_ms, "why": SETTLE_WHY},
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": synth.CONFIGS[args.config]["name"] + ", training step "
                               "(MoEFeedForward forward + autograd backward)",
                   "n_tokens": N, "d_model": d, "d_ff": F, "n_experts": E, "top_k": k,
                   "dropout": args.dropout},
        "accumulation_ms_per_step": ms_acc,
        "dropout_zero_ms_per_step": ms_p0,
        "step_expert_gemm_tflops": (9 * g) / (ms * 1e-3) / 1e12,
        "breakdown": bd,
        "torch_eager_gpu": eager,
        "note": "every stage is this library's HIP kernels; the backward's padded operands "
                "use the packed per-expert layout sized from N k + 384 E rows, so nothing "
                "is read back to the host (no host synchronisation); weight-gradient products in one g5moe_weight_grad launch over per-expert "
                "operands padded to 192-row groups (their zero rows' products count in the "
                "time, not in the FLOP)",
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path; the layer would shard by tokens (data parallel) or by experts, "
              "neither of which is built here.", file=sys.stderr)
        sys.exit(2)
    if args.config in (4, 5):
        out = bench_config4(args) if args.config == 4 else bench_config5(args)
        print(json.dumps(out), flush=True)
        return
    if args.train:
        print(json.dumps(bench_train(args)), flush=True)
        return

    import torch
    from genet5_amd import ops, synth

    dev = torch.device("cuda:0")
    cfg = args.config
    if args.shard is None:
        inp = synth.make_config(cfg, seed=0)
    else:
        inp = synth.make_layer(4550, n_experts=16 if args.shard == "dp8" else 2, top_k=2,
                               seed=0, dtype="bf16")
    N, d = inp.x.shape
    E, F = inp.w_gate.shape[0], inp.w_gate.shape[1]
    k = inp.top_k
    tt = synth.to_torch(inp, dev)
    x, wr, bias = tt["x"], tt["w_router"], tt["bias"]
    wgu = ops.pack_gate_up(tt["w_gate"], tt["w_up"])
    wd = tt["w_down"]
    w_gate_sep, w_up_sep = tt["w_gate"], tt["w_up"]  # the eager-PyTorch comparison's
    del tt
    buf = ops.ForwardBuffers(N, d, F, E, k, x.dtype, dev)
    torch.cuda.synchronize()

    # One step = the whole layer through the C ABI's stage entry points (the
    # same kernels g5moe_forward enqueues), no host synchronisation inside the
    # loop.  HIP events on the stream the stages run on: the timed loop records
    # them only around the two expert GEMMs (indices 1, 2, 3), so the roofline
    # kernel's and the down product's averages come from the timed region
    # itself.  They are TimingEvents (no system-scope fence): with torch's
    # default events the three records cost 0.7 % of the step (0.988 against
    # 0.982 ms per step with TimingEvents and 0.981 with no events, three
    # alternating rounds on one box).
    # The route (router + dispatch) and combine times come from a second loop of the
    # same steps with an event at every stage boundary, run right after.
    import ctypes
    from genet5_amd import _lib
    r = buf.routing
    y_perm = torch.empty((N * k, d), dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev)
    names = ["route", "gate_up", "down", "combine"]
    P = ops._ptr
    shape = buf.shape
    S = ops._stream(dev)
    ws = buf.ws
    every = frozenset(range(len(names) + 1))
    timed_marks = frozenset((1, 2, 3))

    def step(ev=None, marks=every):
        def rec(i):
            if ev is not None and i in marks:
                ev[i].record(stream)
        rec(0)
        # router + dispatch: the router kernel also forms the dispatch's ranks,
        # then one placement kernel
        _lib.call("g5moe_route", P(x), P(wr), P(bias), P(r.topk_idx), P(r.topk_w), None,
                  P(r.counts), P(r.offsets), P(r.perm), P(r.inv_pos), P(ws),
                  ctypes.byref(shape), S)
        rec(1)
        _lib.call("g5moe_expert_gate_up", P(x), P(r.perm), P(r.offsets), P(wgu), P(ws),
                  ctypes.byref(shape), S)
        rec(2)
        _lib.call("g5moe_expert_down", P(r.offsets), P(wd), P(y_perm), P(ws),
                  ctypes.byref(shape), S)
        rec(3)
        _lib.call("g5moe_combine", P(y_perm), P(r.inv_pos), P(r.topk_w), P(buf.y),
                  ctypes.byref(shape), S)
        rec(4)

    events = [[TimingEvent() for _ in range(len(names) + 1)] for _ in range(args.steps)]
    settled = settle(step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i], timed_marks)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1e3 / args.steps
    timed_ms = {n: sum(ev[j].elapsed_time(ev[j + 1]) for ev in events) / args.steps
                for j, n in enumerate(names) if j in timed_marks and j + 1 in timed_marks}
    # the stage breakdown: the same steps with an event at every boundary
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    stage_ms = {n: sum(ev[j].elapsed_time(ev[j + 1]) for ev in events) / args.steps
                for j, n in enumerate(names)}

    flops_gu = 4 * d * F * N * k
    flops_dn = 2 * d * F * N * k
    gu_tflops = flops_gu / (timed_ms["gate_up"] * 1e-3) / 1e12
    dn_tflops = flops_dn / (timed_ms["down"] * 1e-3) / 1e12
    gemm_ms = timed_ms["gate_up"] + timed_ms["down"]
    gemm_tflops = (flops_gu + flops_dn) / (gemm_ms * 1e-3) / 1e12
    router_bytes = N * d * 2 + E * d * 2 + N * k * 8
    combine_bytes = N * k * d * 2 + N * k * 8 + N * d * 2

    # Routing parity on the benchmark inputs (outside the timed regions).
    import oracle
    ref_l = oracle.router_logits(inp.x, inp.w_router, inp.bias)
    ref_i, _ = oracle.topk_gates_c(ref_l, k)
    rc, ro, rp, ri = oracle.dispatch(ref_i, E)
    ops.moe_forward(x, wr, wgu, wd, k, bias=bias, buffers=buf)
    torch.cuda.synchronize()
    routing_exact = bool(
        np.array_equal(r.topk_idx.cpu().numpy(), ref_i)
        and np.array_equal(r.counts.cpu().numpy(), rc)
        and np.array_equal(r.perm.cpu().numpy(), rp)
        and np.array_equal(r.inv_pos.cpu().numpy(), ri))

    # the same layer forward (one g5moe_forward call) captured once in a HIP graph and
    # replayed: how a serving loop would run it (no launch overhead per kernel); a
    # side figure — `value` stays the stage-by-stage loop above
    graph_ms = None
    try:
        gs = torch.cuda.Stream(dev)
        gs.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(gs):
            ops.moe_forward(x, wr, wgu, wd, k, bias=bias, buffers=buf)
        torch.cuda.current_stream(dev).wait_stream(gs)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            ops.moe_forward(x, wr, wgu, wd, k, bias=bias, buffers=buf)
        settle(graph.replay, args.settle_ms)
        for _ in range(args.warmup):
            graph.replay()
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        g0.record()
        for _ in range(args.steps):
            graph.replay()
        g1.record()
        torch.cuda.synchronize()
        graph_ms = g0.elapsed_time(g1) / args.steps
        del graph
    except RuntimeError as exc:  # capture unavailable: report it instead of a number
        graph_ms = f"capture failed: {exc}"

    # the same layer as eager PyTorch code on this GPU (context for `value`)
    y_hip = ops.moe_forward(x, wr, wgu, wd, k, bias=bias, buffers=buf).clone()
    torch.cuda.synchronize()
    torch_gpu = torch_eager_gpu(x, wr, bias, w_gate_sep, w_up_sep, wd, k, y_hip)

    # calibrated HBM bytes per gate|up launch, measured at config 2 (null elsewhere)
    traffic = None
    tf_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                           "gate_up_traffic.json")
    if cfg == 2 and args.shard is None and os.path.exists(tf_path):
        with open(tf_path) as f:
            traffic = json.load(f).get("bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": N / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": settled,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": synth.CONFIGS[cfg]["name"] if args.shard is None else
            ("cfg2 DP-8 shard: 4,550 tok bf16, E=16, top-2 (about 569 rows per expert)"
             if args.shard == "dp8" else
             "cfg2 EP-8 shard: 2 local experts x 4,550 rows (4,550 tok, top-2 of 2)"),
            "n_tokens": N, "d_model": d, "d_ff": F, "n_experts": E, "top_k": k,
            "seed": 0,
        },
        "expert_gemm_tflops": gemm_tflops,
        "expert_gemm_pct_bf16_peak": 100.0 * gemm_tflops / PEAK_BF16_TFLOPS,
        "stage_ms_timed": timed_ms,
        "stage_ms": stage_ms,
        "timing_events": "HIP events created with hipEventDisableSystemFence, on the stages' stream",
        "stage_rates": {
            "gate_up_tflops": gu_tflops,
            "down_tflops": dn_tflops,
            "route_gbs": router_bytes / (stage_ms["route"] * 1e-3) / 1e9,
            "combine_gbs": combine_bytes / (stage_ms["combine"] * 1e-3) / 1e9,
        },
        "roofline": {
            "kernel": "grouped_gemm_persist_kernel<256,256,64,2,3,4,1,false,false,false> (gate|up + SwiGLU)",
            "bound": "mfma",
            "achieved": gu_tflops,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": gu_tflops / PEAK_BF16_TFLOPS,
            "traffic": traffic,
            "flop_per_launch": flops_gu,
        },
        "routing_bit_exact_vs_oracle": routing_exact,
        "graph_ms_per_step": graph_ms,
        "torch_eager_gpu": torch_gpu,
    }
    if args.calibrate_copy:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_cpu_baseline:
        n_cpu = N if args.cpu_sample_tokens <= 0 else min(args.cpu_sample_tokens, N)
        out["cpu_baseline"] = cpu_baseline(inp, n_cpu)
        if cfg == 2 and args.shard is None:
            # the same oracle on the whole of config 1 (2,048 tokens, the reference's
            # CPU-runnable case), beside config 2
            c1 = cpu_baseline(synth.make_config(1, seed=0), 2048)
            out["cpu_baseline"]["config1"] = {k: c1[k] for k in ("value", "unit", "sample")}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
