"""MDLM unmasking driver (config 5's loop): the oracle restatement of
lib/inference/diffusion_engine.py:18-95 pinned by a hand-worked case, and the
harness's vectorised driver compared with it on tie-free confidences, for both
confidence strategies.  CPU only."""
import numpy as np
import pytest
import torch

from genet5_amd.harness import encoder
from oracle import mdlm_oracle

MASK, PAD = 4, 0


class FixedLogits:
    """Target-position logits that do not depend on the ids (vocabulary of 5: 0 = pad,
    4 = mask; the pad and mask columns are the largest so their suppression matters)."""

    def __init__(self, prefix_len):
        t = np.full((6, 5), 0.0)
        t[:, PAD], t[:, MASK] = 10.0, 20.0
        t[0, 1:4] = [5.0, 4.0, 4.0]    # pred 1, margin 1.0,  conf -log(1 + 2/e)          = -0.551
        t[1, 1:4] = [0.0, 8.1, 9.0]    # pred 3, margin 0.9,  conf -log(1 + e^-.9 + e^-9) = -0.341
        t[2, 1:4] = [0.0, 0.0, 7.0]    # pred 3, margin 7.0,  conf                       = -0.002
        t[3, 1:4] = [2.0, 3.5, 0.0]    # pred 2, margin 1.5,  conf                       = -0.226
        t[4, 1:4] = [0.25, 0.0, 2.5]   # pred 3, margin 2.25, conf                       = -0.172
        t[5, 1:4] = [1.0, 1.25, 0.0]   # pred 2, margin 0.25, conf                       = -0.725
        self.table = t
        self.P = prefix_len
        self.calls = 0

    def __call__(self, ids):
        self.calls += 1
        B, L = ids.shape
        out = np.zeros((B, L, 5), dtype=np.float32)
        out[:, self.P:] = self.table
        if isinstance(ids, torch.Tensor):
            return {"logits": torch.from_numpy(out)}
        return {"logits": out}


# Two steps of int(0.4995 * 6) = 2 positions each, then the final fill of the last
# two, which suppresses only the mask token (diffusion_engine.py:88-92), so the pad
# logit (10) wins there.
#   margin:     step 1 {2, 4}, step 2 {3, 0}, fill {1, 5}
#   confidence: step 1 {2, 4}, step 2 {3, 1}, fill {0, 5}
EXPECT = {"margin": [1, PAD, 3, 2, 3, PAD], "confidence": [PAD, 3, 3, 2, 3, PAD]}


@pytest.mark.parametrize("strategy", ["confidence", "margin"])
def test_oracle_hand_worked(strategy):
    assert [mdlm_oracle.step_count(f, 6) for f in mdlm_oracle.linear_unmask_schedule(2)] == [2, 2]
    m = FixedLogits(2)
    stats = {}
    out = mdlm_oracle.diffusion_generate(m, np.array([[3, 1]]), 6, MASK, PAD, 2, strategy, stats)
    assert out.tolist() == [[3, 1] + EXPECT[strategy]]
    assert stats["forwards"] == 3 and m.calls == 3


@pytest.mark.parametrize("strategy", ["confidence", "margin"])
def test_harness_hand_worked(strategy):
    stats = {}
    out = encoder.diffusion_generate(FixedLogits(2), torch.tensor([[3, 1]]), 6, MASK, PAD,
                                     num_steps=2, stats=stats, strategy=strategy)
    assert out.tolist() == [[3, 1] + EXPECT[strategy]]
    assert stats["forwards"] == 3


def test_unknown_strategy_raises():
    with pytest.raises(ValueError, match="strategy"):
        encoder.diffusion_generate(FixedLogits(2), torch.tensor([[3, 1]]), 6, MASK, PAD,
                                   num_steps=2, strategy="entropy")


class StatefulToy:
    """Logits that depend on the current ids: a seeded random table per (row,
    position) plus a term driven by the left neighbour's id, so every unmasking
    changes what later steps see.  Confidences are continuous, hence distinct."""

    def __init__(self, B, L, V, seed):
        rng = np.random.default_rng(seed)
        self.base = (rng.standard_normal((B, L, V)) * 2.0).astype(np.float32)
        self.mix = (rng.standard_normal((V + 1, V)) * 0.75).astype(np.float32)

    def __call__(self, ids):
        is_t = isinstance(ids, torch.Tensor)
        a = ids.cpu().numpy() if is_t else np.asarray(ids)
        left = np.concatenate([np.full((a.shape[0], 1), a.shape[1] * 0), a[:, :-1]], axis=1)
        out = self.base + self.mix[np.clip(left, 0, self.mix.shape[0] - 1)]
        return {"logits": torch.from_numpy(out) if is_t else out}


@pytest.mark.parametrize("strategy", ["confidence", "margin"])
@pytest.mark.parametrize("B,P,T,V,steps,seed", [(3, 10, 40, 50, 4, 0), (2, 7, 64, 33, 16, 1),
                                                 (4, 5, 29, 12, 5, 2)])
def test_harness_matches_oracle_driver(strategy, B, P, T, V, steps, seed):
    mask, pad = V - 1, 0
    model = StatefulToy(B, P + T, V, seed)
    prefix = np.random.default_rng(seed + 100).integers(1, V - 1, (B, P))
    s_ref, s_got = {}, {}
    ref = mdlm_oracle.diffusion_generate(model, prefix, T, mask, pad, steps, strategy, s_ref)
    got = encoder.diffusion_generate(model, torch.from_numpy(prefix), T, mask, pad,
                                     num_steps=steps, stats=s_got, strategy=strategy)
    assert np.array_equal(got.numpy(), ref)
    assert s_got["forwards"] == s_ref["forwards"]
    assert np.array_equal(ref[:, :P], prefix) and not (ref[:, P:] == mask).any()


def test_select_unmask_equals_per_row_topk():
    """The vectorised selection against a per-row topk over the masked positions (the
    reference's loop, diffusion_engine.py:70-82) on distinct confidences."""
    g = torch.Generator().manual_seed(5)
    B, L = 6, 97
    for trial in range(20):
        conf = torch.randperm(B * L, generator=g).view(B, L).float() / 7.0 - 30.0
        is_masked = torch.rand(B, L, generator=g) < 0.6
        is_masked[0] = True
        is_masked[1] = False
        n = torch.minimum(torch.randint(0, L, (B,), generator=g), is_masked.sum(1))
        got = encoder.select_unmask(conf, is_masked, n)
        ref = torch.zeros(B, L, dtype=torch.bool)
        for i in range(B):
            idx = is_masked[i].nonzero(as_tuple=True)[0]
            k = int(n[i])
            if k == 0 or len(idx) == 0:
                continue
            _, top = conf[i, idx].topk(k)
            ref[i, idx[top]] = True
        assert torch.equal(got, ref), trial
