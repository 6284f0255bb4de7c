"""GPU parity of the varlen ALiBi attention kernel (g5moe_attn_varlen_fwd) against
the float64 oracle (oracle.attention_varlen) and a torch fp32 reference, through the
C ABI.

Tolerance (bf16 inputs, fp32 scores and softmax, bf16 probabilities in the output
product as flash-attn does, one bf16 rounding of the output): normwise
max|err| / max|ref| <= 1e-2 and mean|err| / mean|ref| <= 4e-3 per case.  The bf16
rounding of the output alone costs a mean of about 1e-3; of the probabilities about
as much again."""
import math

import numpy as np
import pytest
import torch

import oracle
from genet5_amd import attention, ops
from genet5_amd.attention import alibi_slopes

pytestmark = pytest.mark.gpu

MAX_TOL = 1e-2
MEAN_TOL = 4e-3


def make(cu, H, Hkv, seed, scale=1.0, dev="cuda:0"):
    g = torch.Generator(device="cpu").manual_seed(seed)
    T = cu[-1]
    q = (torch.randn(T, H, 64, generator=g) * scale).to(torch.bfloat16)
    k = (torch.randn(T, Hkv, 64, generator=g) * scale).to(torch.bfloat16)
    v = torch.randn(T, Hkv, 64, generator=g).to(torch.bfloat16)
    return q.to(dev), k.to(dev), v.to(dev)


def errs(got, ref, rows=None):
    got = got.float().cpu().numpy().astype(np.float64)
    if rows is not None:
        got, ref = got[rows], ref[rows]
    e = np.abs(got - ref)
    return e.max() / np.abs(ref).max(), e.mean() / np.abs(ref).mean()


def run(q, k, v, cu, slopes, lse=False):
    dev = q.device
    cu_t = torch.tensor(cu, dtype=torch.int32, device=dev)
    sl = None if slopes is None else torch.tensor(slopes, dtype=torch.float32, device=dev)
    L = max(b - a for a, b in zip(cu[:-1], cu[1:])) if len(cu) > 1 else 0
    return attention.attn_varlen_fwd(q, k, v, cu_t, L, 1.0 / 8.0, sl, return_lse=lse)


CASES = [
    ([0, 1], 12, 12, True),
    ([0, 5, 68, 132, 195], 12, 12, True),
    ([0, 64, 128, 256], 12, 12, True),
    ([0, 127, 256, 385, 685], 12, 12, True),
    ([0, 63, 129, 1129], 12, 12, False),
    ([0, 300, 301, 901], 12, 4, True),
    ([0, 200, 440], 8, 1, True),
]


@pytest.mark.parametrize("cu,H,Hkv,use_alibi", CASES)
@pytest.mark.parametrize("scale", [1.0, 3.0])
def test_attention_matches_oracle(cuda_device, cu, H, Hkv, use_alibi, scale):
    print(f"attn case cu={cu} H={H} Hkv={Hkv} alibi={use_alibi} scale={scale}", flush=True)
    q, k, v = make(cu, H, Hkv, seed=len(cu) * 7 + H, scale=scale)
    slopes = alibi_slopes(H) if use_alibi else None
    out, lse = run(q, k, v, cu, slopes, lse=True)
    torch.cuda.synchronize()
    ref, ref_lse = oracle.attention_varlen(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                           v.float().cpu().numpy(), cu, 1.0 / 8.0, slopes,
                                           return_lse=True)
    mx, mean = errs(out, ref)
    print(f"  max_rel={mx:.2e} mean_rel={mean:.2e}", flush=True)
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (mx, mean)
    # lse: fp32 scores against float64
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=0, atol=2e-4 * scale ** 2 + 1e-5)


def test_attention_deterministic_and_strided_views(cuda_device):
    cu = [0, 100, 333, 334, 800]
    T, H = cu[-1], 12
    g = torch.Generator(device="cpu").manual_seed(11)
    qkv = torch.randn(T, 3, H, 64, generator=g).to(torch.bfloat16).to(cuda_device)
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]  # token stride 3 * 768
    sl = alibi_slopes(H)
    a = run(q, k, v, cu, sl)
    b = run(q, k, v, cu, sl)
    c = run(q.contiguous(), k.contiguous(), v.contiguous(), cu, sl)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)
    ref = oracle.attention_varlen(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                  v.float().cpu().numpy(), cu, 1.0 / 8.0, sl)
    mx, mean = errs(a, ref)
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (mx, mean)


def test_attention_empty_sequences_and_larger_max_seqlen(cuda_device):
    cu = [0, 0, 37, 37, 100]
    q, k, v = make(cu, 12, 12, seed=3)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda_device)
    sl = torch.tensor(alibi_slopes(12), dtype=torch.float32, device=cuda_device)
    out = attention.attn_varlen_fwd(q, k, v, cu_t, 500, 0.125, sl)  # max_seqlen > every length
    torch.cuda.synchronize()
    ref = oracle.attention_varlen(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                  v.float().cpu().numpy(), cu, 0.125, alibi_slopes(12))
    mx, mean = errs(out, ref)
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (mx, mean)
    # no sequences at all: nothing is launched
    e = attention.attn_varlen_fwd(q[:0], k[:0], v[:0], cu_t[:1], 0, 0.125, sl)
    assert e.shape == (0, 12, 64)


def test_attention_config5_rows_against_oracle(cuda_device):
    """Config 5's shape (8 sequences x 4,550 tokens, 12 heads): every head, a fixed set
    of query rows per sequence (block and diagonal boundaries, both ends), against the
    float64 oracle over all keys."""
    B, L, H = 8, 4550, 12
    cu = [i * L for i in range(B + 1)]
    q, k, v = make(cu, H, H, seed=5)
    sl = alibi_slopes(H)
    out = run(q, k, v, cu, sl)
    torch.cuda.synchronize()
    local = np.array([0, 1, 31, 32, 63, 64, 127, 128, 2047, 2048, 2275, 4479, 4480, 4548, 4549])
    rows = np.concatenate([s * L + local for s in (0, 3, 7)])
    ref = oracle.attention_varlen(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                  v.float().cpu().numpy(), cu, 1.0 / 8.0, sl, rows=rows)
    mx, mean = errs(out, ref, rows)
    print(f"cfg5 rows: max_rel={mx:.2e} mean_rel={mean:.2e}", flush=True)
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (mx, mean)


def test_attention_against_torch_fp32_full_sequence(cuda_device):
    """One config-5 sequence (4,550 tokens, 12 heads) against torch fp32 attention with
    the ALiBi bias as an explicit mask, all rows."""
    L, H = 4550, 12
    q, k, v = make([0, L], H, H, seed=9)
    sl = alibi_slopes(H)
    out = run(q, k, v, [0, L], sl)
    pos = torch.arange(L, device=cuda_device, dtype=torch.float32)
    dist = (pos[:, None] - pos[None, :]).abs()
    slopes = torch.tensor(sl, device=cuda_device)
    ref = torch.empty(L, H, 64, device=cuda_device)
    for h in range(H):
        s = (q[:, h].float() @ k[:, h].float().T) / 8.0 - slopes[h] * dist
        ref[:, h] = torch.softmax(s, dim=-1) @ v[:, h].float()
    torch.cuda.synchronize()
    mx, mean = errs(out, ref.double().cpu().numpy())
    print(f"torch fp32: max_rel={mx:.2e} mean_rel={mean:.2e}", flush=True)
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (mx, mean)


def test_flash_attn_func_and_module(cuda_device):
    B, L, H = 3, 200, 12
    q, k, v = make([0, B * L], H, H, seed=13)
    sl = torch.tensor(alibi_slopes(H), dtype=torch.float32, device=cuda_device)
    fixed = attention.flash_attn_func(q.view(B, L, H, 64), k.view(B, L, H, 64),
                                      v.view(B, L, H, 64), alibi_slopes=sl)
    cu = torch.tensor([0, L, 2 * L, 3 * L], dtype=torch.int32, device=cuda_device)
    var = attention.flash_attn_varlen_func(q, k, v, cu, cu, L, L, alibi_slopes=sl)
    torch.cuda.synchronize()
    assert torch.equal(fixed.view(B * L, H, 64), var)

    cfg = attention.FlashAttentionConfig(embed_dim=768, num_heads=12)
    m = attention.FlashAttention(cfg).to(cuda_device).to(torch.bfloat16).eval()
    h = torch.randn(1, 3 * L, 768, device=cuda_device).to(torch.bfloat16)
    with torch.no_grad():
        out, none = m(h, cu_seqlens=cu, max_seqlen=L)
        out_b, _ = m(h.view(3, L, 768))
        # reference composition: the module's own inference projections (one fused
        # q|k|v product on ops.linear), fp32 attention per sequence
        qkv = ops.linear(h.reshape(3 * L, 768), m.qkv_weight())
        qq = qkv[:, :768].view(3 * L, 12, 64)
        kk = qkv[:, 768:1536].view(3 * L, 12, 64)
        vv = qkv[:, 1536:].view(3 * L, 12, 64)
    assert none is None and out.shape == h.shape
    assert torch.equal(out.view(3, L, 768), out_b)
    ref = oracle.attention_varlen(qq.float().cpu().numpy(), kk.float().cpu().numpy(),
                                  vv.float().cpu().numpy(), [0, L, 2 * L, 3 * L], 1.0 / 8.0,
                                  alibi_slopes(12))
    attn = attention.attn_varlen_fwd(qq, kk, vv, cu, L, 1.0 / 8.0, sl)
    mx, mean = errs(attn, ref)
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (mx, mean)
    with torch.no_grad():
        ref_out = ops.linear(attn.reshape(3 * L, 768), m.o.weight).view(1, 3 * L, 768)
    assert torch.equal(out, ref_out)
    # with a gradient the projections are the nn.Linear modules (hipBLASLt): the
    # same values up to the bf16 rounding of another fp32 summation order
    with torch.enable_grad():
        hg = h.clone().requires_grad_(True)
        try:
            out_g, _ = m(hg, cu_seqlens=cu, max_seqlen=L)
        except NotImplementedError:
            out_g = None  # an inference-only kernel may refuse the autograd path
    if out_g is not None:
        d = (out_g.detach().float() - out.float()).abs()
        assert d.max().item() <= 5e-2 * out.float().abs().max().item()


def test_harness_attention_backends_agree(cuda_device):
    """The config-5 harness's attention sublayer: HIP backend against the PyTorch
    reference composition (SDPA with the explicit bias, run here in fp32), packed and
    batched inputs."""
    from genet5_amd.harness import encoder
    torch.manual_seed(17)
    attn = encoder.ALiBiSelfAttention(768, 12).to(cuda_device)
    with torch.no_grad():
        for p in attn.parameters():
            p.normal_(0, 0.05)
    h = torch.randn(1, 700, 768, device=cuda_device)
    cu = torch.tensor([0, 250, 251, 700])
    with torch.no_grad():
        attn_bf = attn.to(torch.bfloat16)
        got_packed = attn_bf(h.to(torch.bfloat16), cu).float()
        got_batch = attn_bf(h.to(torch.bfloat16).view(2, 350, 768)).float()
        attn_bf.backend = "torch"
        attn32 = attn_bf.float()
        hb = h.to(torch.bfloat16).float()
        ref_packed = attn32(hb, cu)
        ref_batch = attn32(hb.view(2, 350, 768))
    for got, ref in ((got_packed, ref_packed), (got_batch, ref_batch)):
        mx, mean = errs(got, ref.double().cpu().numpy())
        print(f"harness attention hip vs torch: max_rel={mx:.2e} mean_rel={mean:.2e}", flush=True)
        assert mx <= 2e-2 and mean <= 8e-3, (mx, mean)


@pytest.mark.parametrize("scale", [0.3, 1.0, 3.0])
def test_key_bounds_equal_dense(cuda_device, scale):
    """Config-5-shaped inputs with ALiBi, the kernel with key-norm bounds (block
    skipping, and the reference-max loop where the bounds allow) against the plain
    online-softmax kernel over every block.

    scale 3.0: the bounds are too loose for the reference-max loop (|s| * sc up to
    ~130), so both runs take the online loop and differ only by the skipped blocks,
    which carry less than 2^-51 of each row's mass: outputs and lse equal bit for bit.
    scale 0.3 / 1.0: the reference-max loop runs (its bf16 probabilities are scaled
    by 2^(m - mref) against the online loop's, so the runs are not bit-equal; that
    they differ shows the loop ran); both agree within the rounding of the
    probabilities, and with the float64 oracle on sampled rows."""
    B, L, H = 8, 4550, 12
    cu = [i * L for i in range(B + 1)]
    q, k, v = make(cu, H, H, seed=21, scale=scale)
    cu_t = torch.tensor(cu, dtype=torch.int32, device=cuda_device)
    sl = torch.tensor(alibi_slopes(H), dtype=torch.float32, device=cuda_device)
    out_s, lse_s = attention.attn_varlen_fwd(q, k, v, cu_t, L, 0.125, sl, return_lse=True,
                                             key_bounds=True)
    out_d, lse_d = attention.attn_varlen_fwd(q, k, v, cu_t, L, 0.125, sl, return_lse=True,
                                             key_bounds=False)
    torch.cuda.synchronize()
    if scale >= 3.0:
        assert torch.equal(out_s, out_d)
        assert torch.equal(lse_s, lse_d)
        return
    assert not torch.equal(out_s, out_d)
    a, b = out_s.float(), out_d.float()
    mx = ((a - b).abs().max() / b.abs().max()).item()
    mean = ((a - b).abs().mean() / b.abs().mean()).item()
    print(f"key bounds vs dense scale={scale}: max_rel={mx:.2e} mean_rel={mean:.2e}", flush=True)
    assert mx <= 1e-2 and mean <= 2e-3, (mx, mean)
    assert (lse_s - lse_d).abs().max().item() <= 1e-4
    local = np.array([0, 1, 63, 64, 2047, 2275, 4480, 4549])
    rows = np.concatenate([s_ * L + local for s_ in (0, 5)])
    ref = oracle.attention_varlen(q.float().cpu().numpy(), k.float().cpu().numpy(),
                                  v.float().cpu().numpy(), cu, 0.125, alibi_slopes(H), rows=rows)
    mx, mean = errs(out_s, ref, rows)
    assert mx <= MAX_TOL and mean <= MEAN_TOL, (mx, mean)


@pytest.mark.parametrize("kv_heads", [12, 4])
def test_flash_attention_module_fused_projections(cuda_device, kv_heads):
    """The drop-in FlashAttention module in inference (one fused q|k|v product and
    the o product on ops.linear), with and without GQA, against the same module
    with its nn.Linear projections (forced): equal up to the bf16 rounding of the
    projections' different fp32 summation orders."""
    print(f"FlashAttention fused projections kv_heads={kv_heads}", flush=True)
    torch.manual_seed(23)
    cfg = attention.FlashAttentionConfig(embed_dim=768, num_heads=12, num_kv_heads=kv_heads)
    m = attention.FlashAttention(cfg).to(cuda_device).to(torch.bfloat16).eval()
    h = torch.randn(2, 1000, 768, device=cuda_device).to(torch.bfloat16)
    with torch.no_grad():
        assert m._fused_projections(h)
        fused, _ = m(h)
        m._fused_projections = lambda x: False
        plain, _ = m(h)
    torch.cuda.synchronize()
    d = (fused.float() - plain.float()).abs()
    ref = plain.float().abs()
    assert d.max().item() <= 2e-2 * ref.max().item()
    assert d.mean().item() <= 4e-3 * ref.mean().item()
