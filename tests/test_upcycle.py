"""Dense -> MoE checkpoint upcycling (genet5_amd.upcycle), on the CPU.

The dense checkpoint is built with the reference's key layout (GeneT5.save,
lib/model/genet5.py:71-84: {"embed", "encoder", "lm_head"}; encoder keys
layers.{i}.self_attn.{q,k,v,o}.weight, layers.{i}.norm{1,2}.weight,
layers.{i}.ff.{wi_0,wi_1,wo}.weight, final_norm.weight), saved with torch.save
and read back with weights_only=True."""
import warnings

import pytest
import torch

from genet5_amd import upcycle
from genet5_amd.harness import encoder

D, F, H, V, LAYERS, E = 128, 256, 4, 64, 2, 4


def dense_checkpoint(seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    enc = {}
    for i in range(LAYERS):
        for p in "qkvo":
            enc[f"layers.{i}.self_attn.{p}.weight"] = r(D, D)
        enc[f"layers.{i}.norm1.weight"] = r(D)
        enc[f"layers.{i}.norm2.weight"] = r(D)
        enc[f"layers.{i}.ff.wi_0.weight"] = r(F, D)
        enc[f"layers.{i}.ff.wi_1.weight"] = r(F, D)
        enc[f"layers.{i}.ff.wo.weight"] = r(D, F)
    enc["final_norm.weight"] = r(D)
    emb = r(V, D)
    return {"embed": {"weight": emb}, "encoder": enc, "lm_head": {"weight": emb.clone()}}


def model():
    return encoder.GeneT5MoE(vocab_size=V, embed_dim=D, num_layers=LAYERS, num_heads=H,
                             ff_dim=F, num_experts=E, top_k=2)


def test_upcycled_experts_are_copies_of_the_dense_ffn(tmp_path):
    ck = dense_checkpoint()
    path = tmp_path / "dense.pt"
    torch.save(ck, path)
    m = model()
    rep = upcycle.load_upcycled(m, path)
    assert rep.clean and rep.upcycled_layers == [0, 1]
    enc = ck["encoder"]
    for i, layer in enumerate(m.layers):
        for e in range(E):
            assert torch.equal(layer.ff.w_gate[e], enc[f"layers.{i}.ff.wi_0.weight"])
            assert torch.equal(layer.ff.w_up[e], enc[f"layers.{i}.ff.wi_1.weight"])
            assert torch.equal(layer.ff.w_down[e], enc[f"layers.{i}.ff.wo.weight"])
        assert torch.equal(layer.self_attn.q.weight, enc[f"layers.{i}.self_attn.q.weight"])
        assert torch.equal(layer.norm2.weight, enc[f"layers.{i}.norm2.weight"])
    assert torch.equal(m.final_norm.weight, enc["final_norm.weight"])
    assert torch.equal(m.embed.weight, ck["embed"]["weight"])


def test_router_init_is_seeded_and_per_layer():
    a = upcycle.upcycle_encoder_state_dict(dense_checkpoint()["encoder"], E, seed=3)
    b = upcycle.upcycle_encoder_state_dict(dense_checkpoint()["encoder"], E, seed=3)
    c = upcycle.upcycle_encoder_state_dict(dense_checkpoint()["encoder"], E, seed=4)
    r0, r1 = a["layers.0.ff.router.weight"], a["layers.1.ff.router.weight"]
    assert r0.shape == (E, D) and torch.equal(r0, b["layers.0.ff.router.weight"])
    assert not torch.equal(r0, r1) and not torch.equal(r0, c["layers.0.ff.router.weight"])
    assert 0.003 < float(r0.std()) < 0.012  # N(0, 0.006^2)


def test_decoder_key_is_accepted():
    ck = dense_checkpoint()
    ck["decoder"] = ck.pop("encoder")
    assert upcycle.load_upcycled(model(), ck).clean


def test_unexpected_key_is_loud():
    ck = dense_checkpoint()
    ck["encoder"]["layers.0.attn_typo.weight"] = torch.zeros(3)
    with pytest.raises(KeyError, match="unexpected.*layers.0.attn_typo.weight"):
        upcycle.load_upcycled(model(), ck)
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        rep = upcycle.load_upcycled(model(), ck, strict=False)
    assert rep.unexpected == ["layers.0.attn_typo.weight"]
    assert any("attn_typo" in str(x.message) for x in w)


def test_missing_key_is_loud():
    ck = dense_checkpoint()
    del ck["encoder"]["layers.1.norm1.weight"]
    with pytest.raises(KeyError, match="missing.*layers.1.norm1.weight"):
        upcycle.load_upcycled(model(), ck)


def test_shape_mismatch_is_loud():
    ck = dense_checkpoint()
    ck["encoder"]["final_norm.weight"] = torch.zeros(D + 1)
    with pytest.raises(KeyError, match="shape-mismatched.*final_norm.weight"):
        upcycle.load_upcycled(model(), ck)


def test_partial_or_inconsistent_dense_ffn_raises():
    enc = dense_checkpoint()["encoder"]
    del enc["layers.0.ff.wi_1.weight"]
    with pytest.raises(ValueError, match=r"layer 0.*missing \['wi_1'\]"):
        upcycle.upcycle_encoder_state_dict(enc, E)
    enc = dense_checkpoint()["encoder"]
    enc["layers.1.ff.wo.weight"] = torch.zeros(F, D)
    with pytest.raises(ValueError, match="layer 1: inconsistent"):
        upcycle.upcycle_encoder_state_dict(enc, E)


def test_missing_checkpoint_part_raises():
    ck = dense_checkpoint()
    del ck["lm_head"]
    with pytest.raises(KeyError, match="lm_head"):
        upcycle.load_upcycled(model(), ck)
