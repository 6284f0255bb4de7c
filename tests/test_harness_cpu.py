"""CPU checks of the config-4/5 harness pieces that do not need the GPU:
ALiBi slopes and attention, packed attention, RMSNorm, the unmasking schedule and
driver (with a stand-in model), and the config-4 input packing."""
import math

import numpy as np
import pytest
import torch

from genet5_amd.harness import blocks, encoder


def test_alibi_slopes_closed_form():
    assert encoder.alibi_slopes(8) == [2.0 ** -(i + 1) for i in range(8)]
    s16 = [2.0 ** (-(i + 1) / 2) for i in range(16)]
    assert np.allclose(encoder.alibi_slopes(16), s16)
    # 12 heads: the 8-head slopes then every other 16-head slope (Press et al. 2022)
    assert np.allclose(encoder.alibi_slopes(12), [2.0 ** -(i + 1) for i in range(8)] + s16[0::2][:4])


def explicit_attention(x, attn):
    B, L, D = x.shape
    H, hd = attn.num_heads, attn.head_dim
    q = (x @ attn.q.weight.T).view(B, L, H, hd).permute(0, 2, 1, 3).double()
    k = (x @ attn.k.weight.T).view(B, L, H, hd).permute(0, 2, 1, 3).double()
    v = (x @ attn.v.weight.T).view(B, L, H, hd).permute(0, 2, 1, 3).double()
    out = torch.zeros(B, H, L, hd, dtype=torch.float64)
    for h in range(H):
        s = attn.slopes[h].item()
        for i in range(L):
            sc = torch.einsum("bd,bjd->bj", q[:, h, i], k[:, h]) / math.sqrt(hd)
            sc = sc - s * torch.abs(torch.arange(L, dtype=torch.float64) - i)
            out[:, h, i] = torch.einsum("bj,bjd->bd", torch.softmax(sc, -1), v[:, h])
    return (out.permute(0, 2, 1, 3).reshape(B, L, D).float()) @ attn.o.weight.T


def test_alibi_attention_matches_explicit_softmax():
    torch.manual_seed(0)
    attn = encoder.ALiBiSelfAttention(32, 4, backend="torch")
    x = torch.randn(2, 9, 32)
    got = attn(x)
    ref = explicit_attention(x, attn)
    assert torch.allclose(got, ref, atol=2e-5, rtol=1e-4)
    # bias is symmetric and zero on the diagonal
    b = attn.alibi_bias(9, torch.float32, x.device)[0]
    assert torch.equal(b, b.transpose(-1, -2)) and (b.diagonal(dim1=-2, dim2=-1) == 0).all()


def test_packed_attention_is_block_diagonal():
    torch.manual_seed(1)
    attn = encoder.ALiBiSelfAttention(32, 4, backend="torch")
    a, b = torch.randn(1, 5, 32), torch.randn(1, 7, 32)
    packed = attn(torch.cat([a, b], 1), torch.tensor([0, 5, 12]))
    assert torch.allclose(packed[:, :5], attn(a), atol=1e-6)
    assert torch.allclose(packed[:, 5:], attn(b), atol=1e-6)


def test_rmsnorm_textbook():
    n = blocks.RMSNorm(16)
    with torch.no_grad():
        n.weight.copy_(torch.linspace(0.5, 2.0, 16))
    x = torch.randn(4, 16, dtype=torch.float64).float()
    ref = x.double() / torch.sqrt((x.double() ** 2).mean(-1, keepdim=True) + 1e-6) * n.weight.double()
    assert torch.allclose(n(x).double(), ref, atol=1e-6)
    xb = x.to(torch.bfloat16)
    assert n(xb).dtype == torch.bfloat16


def test_unmask_schedule():
    fr = encoder.linear_unmask_schedule(16)
    assert len(fr) == 16 and abs(sum(fr) - (1 - 1e-3)) < 1e-6
    assert int(fr[0] * 2275) == 142   # 142 tokens per step, 3 left -> 17th pass


class ToyModel:
    """Logits that prefer token (position * 7) % V at each position, with position-dependent confidence."""

    def __init__(self, V):
        self.V = V

    def __call__(self, ids):
        B, L = ids.shape
        pos = torch.arange(L)
        logits = torch.zeros(B, L, self.V)
        logits[:, pos, (pos * 7) % self.V] = 1.0 + pos.float() / L
        return {"logits": logits}


def test_diffusion_generate_toy():
    V, mask, pad = 50, 49, 0
    prefix = torch.randint(1, 40, (3, 10))
    stats = {}
    out = encoder.diffusion_generate(ToyModel(V), prefix, 40, mask, pad, num_steps=4, stats=stats)
    assert torch.equal(out[:, :10], prefix)
    assert not (out[:, 10:] == mask).any()
    pos = torch.arange(10, 50)
    expect = (pos * 7) % V
    expect[expect == pad] = -1  # pad is suppressed: the argmax moves elsewhere
    ok = (out[0, 10:] == expect) | (expect == -1)
    assert ok.all()
    assert stats["forwards"] == 5  # 4 steps leave int(0.24975*40)*4 = 36 unmasked -> final fill


def test_config4_packing():
    c = blocks.make_config4()
    lens = np.diff(c.cu_seqlens)
    assert c.cu_seqlens[-1] == 45500 and c.x.shape == (1, 45500, 768)
    assert (lens[:-1] >= 1000).all() and (lens <= 9000).all()
    assert c.layer_seeds == list(range(12))


def test_attention_backend_choice_is_explicit():
    import pytest
    with pytest.raises(ValueError, match="backend"):
        encoder.ALiBiSelfAttention(32, 4, backend="eager")
    m = encoder.GeneT5MoE(vocab_size=64, embed_dim=128, num_layers=2, num_heads=2, ff_dim=256)
    assert all(l.self_attn.backend == "hip" for l in m.layers)
    m.set_attention_backend("torch")
    assert all(l.self_attn.backend == "torch" for l in m.layers)
    # the HIP backend never runs on CPU tensors (no silent fallback)
    m.set_attention_backend("hip")
    with pytest.raises(RuntimeError, match="GPU only"), torch.no_grad():
        m.layers[0].self_attn(torch.zeros(1, 4, 128))
    # slopes stay fp32 through a bf16 cast of the model
    m = m.to(torch.bfloat16)
    assert m.layers[0].self_attn.slopes.dtype == torch.float32
    assert m.layers[0].self_attn.slopes[1].item() == 2.0 ** -8
