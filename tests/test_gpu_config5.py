"""Config 5 at its workload: the full 12-layer GeneT5-shaped encoder (d 768, 12 heads,
vocab 4,096, HIP ALiBi attention, HIP MoE with 16 experts top-2 in every layer,
fused blocks) on 8 sequences of 4,550 tokens (2,275 prefix + 2,275 [MASK]), and the
16-step MDLM unmasking run (lib/inference/diffusion_engine.py:18-95) on it.

One forward of the unmasking run's first input with hooks; for each of the 12
layers, on the inputs that forward actually produced:
  * attention: the hooked attention output is the HIP kernel's core output
    through the o projection (the module's own projection, ops.linear: recomputed
    bit for bit), and that core output is
    within the attention bar of the float64 oracle (oracle.attention_varlen) on
    sampled query rows of every sequence (block and diagonal boundaries, both
    ends, random rows);
  * MoE half (fused: add + RMSNorm + router, dispatch, experts, combine into the
    residual): the normed and sum rows, the routing (indices, counts, offsets,
    permutation) and the block output bit-exact against the C oracle;
  * the MoE output within 2e-2 / 2e-3 of the oracle's bf16-storage mode on a
    fixed sample of 1,536 rows.
Then the unmasking run twice: 17 forwards, identical outputs, the prefix
untouched, no [MASK] left."""
import numpy as np
import pytest
import torch

import oracle
from genet5_amd import attention, ops
from genet5_amd.harness import encoder
from test_gpu_harness import bits, normwise

pytestmark = pytest.mark.gpu

B, P, T = 8, 2275, 2275
L = P + T
D, H, HD = 768, 12, 64
MASK, PAD = 4095, 0


def full_model(dev):
    """The model bench.py --config 5 runs: N(0, 0.02) weights, seed 0, bf16, eval."""
    torch.manual_seed(0)
    model = encoder.GeneT5MoE().to(dev)
    with torch.no_grad():
        for p in model.parameters():
            if p.dim() >= 2:
                p.normal_(0, 0.02)
    return model.to(torch.bfloat16).eval()


def prefix_ids():
    g = torch.Generator(device="cpu").manual_seed(0)
    return torch.randint(1, 4095, (B, P), generator=g)


def attention_rows(rng):
    local = np.array([0, 1, 63, 64, 127, 128, 2274, 2275, 4479, 4480, 4549])
    return np.concatenate([s * L + np.unique(np.concatenate([local, rng.integers(0, L, 8)]))
                           for s in range(B)])


def test_config5_full_size_per_layer(cuda_device):
    model = full_model(cuda_device)
    ids = torch.cat([prefix_ids(), torch.full((B, T), MASK)], 1).to(cuda_device)
    ins, attn_in, attn_out, outs = [], [], [], []
    hooks = []
    def keep_attention(m, a, o):  # returns None: the module's output is unchanged
        attn_in.append(a[0])
        attn_out.append(o)

    for layer in model.layers:
        hooks.append(layer.register_forward_pre_hook(lambda m, a: ins.append(a[0])))
        hooks.append(layer.self_attn.register_forward_hook(keep_attention))
        hooks.append(layer.register_forward_hook(lambda m, a, o: outs.append(o)))
    with torch.no_grad():
        logits = model(ids)["logits"]
    for h in hooks:
        h.remove()
    torch.cuda.synchronize()
    assert logits.shape == (B, L, 4096) and torch.isfinite(logits.float()).all()
    assert len(outs) == len(model.layers) == 12
    rng = np.random.default_rng(0)
    rows = attention_rows(rng)
    moe_rows = np.sort(rng.choice(B * L, 1536, replace=False))
    cu = torch.arange(0, (B + 1) * L, L, dtype=torch.int32, device=cuda_device)
    cu_np = [i * L for i in range(B + 1)]
    for li, layer in enumerate(model.layers):
        print(f"config5 full layer {li}", flush=True)
        sa = layer.self_attn
        with torch.no_grad():
            # attention core on this layer's actual normed input
            qkv = sa.project(attn_in[li].reshape(B * L, D), sa.qkv_weight()).view(B * L, 3, H,
                                                                                   HD)
            q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
            core = attention.flash_attn_varlen_func(q, k, v, cu, cu, L, L,
                                                    softmax_scale=1.0 / 8.0,
                                                    alibi_slopes=sa.slopes_on(cuda_device))
            assert torch.equal(sa.project(core.view(B * L, D), sa.o.weight).view(B, L, D),
                               attn_out[li])
        sl = np.asarray(sa.slopes, np.float64)
        ref_a = oracle.attention_varlen(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                        v.float().cpu().numpy(), cu_np, 1.0 / 8.0, sl, rows=rows)
        got_a = core.float().cpu().numpy().astype(np.float64)[rows]
        mx, mean = normwise(got_a, ref_a[rows])
        print(f"  attention rows: max_rel={mx:.3e} mean_rel={mean:.3e}", flush=True)
        assert mx <= 1e-2 and mean <= 4e-3, (li, mx, mean)

        # MoE half, fused, on the block's input and attention output
        h2 = ins[li].reshape(-1, D)
        a2 = attn_out[li].reshape(-1, D).contiguous()
        nw = layer.norm2.weight.detach().float().contiguous()
        ff = layer.ff
        with torch.no_grad():
            normed, ssum, idx, w = ops.add_rmsnorm_router(h2, nw, 1e-6,
                                                          ff.router.weight.contiguous(), 2,
                                                          x_add=a2)
            counts, offsets, perm, inv_pos = ops.dispatch(idx, 16, D)
            wgu, wd = ff._expert_weights()
            y_perm = ops.expert_swiglu(normed, perm, offsets, wgu, wd, 2)
            y = ops.combine(y_perm, inv_pos, w, torch.bfloat16)
        torch.cuda.synchronize()
        n_ref, s_ref = oracle.add_rmsnorm(bits(h2), nw.cpu().numpy(), 1e-6, bits(a2))
        np.testing.assert_array_equal(bits(normed), n_ref)
        np.testing.assert_array_equal(bits(ssum), s_ref)
        wr = bits(ff.router.weight)
        ref_i, _ = oracle.topk_gates_c(oracle.router_logits(n_ref, wr), 2)
        np.testing.assert_array_equal(idx.cpu().numpy(), ref_i)
        c_ref, o_ref, p_ref, ip_ref = oracle.dispatch_c(ref_i, 16)
        np.testing.assert_array_equal(counts.cpu().numpy(), c_ref)
        np.testing.assert_array_equal(offsets.cpu().numpy(), o_ref)
        np.testing.assert_array_equal(perm.cpu().numpy(), p_ref)
        np.testing.assert_array_equal(inv_pos.cpu().numpy(), ip_ref)
        out_ref = oracle.combine_c(bits(y_perm), inv_pos.cpu().numpy(), w.cpu().numpy(), s_ref,
                                   1.0)
        np.testing.assert_array_equal(bits(outs[li].reshape(-1, D)), out_ref)
        ref = oracle.moe_forward(n_ref[moe_rows], wr, bits(ff.w_gate), bits(ff.w_up),
                                 bits(ff.w_down), 2, storage="bf16")
        np.testing.assert_array_equal(ref["topk_idx"], ref_i[moe_rows])
        mx, mean = normwise(y.float().cpu().numpy()[moe_rows], ref["y"])
        print(f"  moe rows: max_rel={mx:.3e} mean_rel={mean:.3e}", flush=True)
        assert mx <= 2e-2 and mean <= 2e-3, (li, mx, mean)


def test_config5_full_size_unmasking_run(cuda_device):
    model = full_model(cuda_device)
    prefix = prefix_ids().to(cuda_device)
    st1, st2 = {}, {}
    out1 = encoder.diffusion_generate(model, prefix, T, MASK, PAD, num_steps=16, stats=st1)
    out2 = encoder.diffusion_generate(model, prefix, T, MASK, PAD, num_steps=16, stats=st2)
    torch.cuda.synchronize()
    assert st1["forwards"] == st2["forwards"] == 17
    assert torch.equal(out1, out2)
    assert out1.shape == (B, L) and torch.equal(out1[:, :P], prefix)
    assert not (out1[:, P:] == MASK).any()
