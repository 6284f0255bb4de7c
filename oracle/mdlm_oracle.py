"""CPU restatement of GeneT5's MDLM unmasking driver — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, as the checker.

diffusion_generate(model, prefix_ids, target_len, mask_token_id, pad_token_id,
                   num_steps, strategy)
select_step(logits, masked, want, strategy)
    One step's predictions, confidences and chosen positions (the driver's body).
    The reference's diffusion_generate (lib/inference/diffusion_engine.py:18-95)
    at temperature 0, one row at a time, in numpy float64:
      * the target starts fully masked after the prefix (:33-35);
      * the schedule is linear_unmask_schedule (:5-15): differences of
        torch.linspace(1.0, 1e-3, T + 1) — the same library call, since the
        fractions are defined by its float32 values;
      * each step runs the model, suppresses the mask and pad tokens (:44-46),
        takes the argmax prediction (:53), and a per-position confidence: the
        log-softmax of the prediction ("confidence", :58-60) or the gap between
        the two largest logits ("margin", :54-56); unmasked positions get -inf
        (:62);
      * the count of this step is the float32 product frac * target_len
        truncated (:65-66), capped by the positions still masked (:67);
      * per row, the count largest confidences among the still-masked positions
        are unmasked with their predictions (:70-82, a per-row topk);
      * a final pass fills whatever is still masked with the argmax (:85-93).
    `model(ids)` returns {"logits": array or tensor [B, L, V]}; it is called
    with an int64 numpy array of the current ids.
    Pins (tests/test_mdlm_driver.py): a hand-worked 1-row case whose every
    step's counts and choices are written out; the fully-masked-start /
    prefix-kept / no-mask-left invariants; the forward count of the schedule
    (T forwards plus the final fill when the truncated counts leave masks).
    On tie-free confidences the per-row topk selection is a set, independent of
    how ties would be broken, which is what the harness is compared on.
"""
from __future__ import annotations

from typing import Callable, List

import numpy as np


def linear_unmask_schedule(num_steps: int, eps: float = 1e-3) -> List[float]:
    """Fractions t[i] - t[i+1] of t = torch.linspace(1, eps, T + 1) in float32
    (lib/inference/diffusion_engine.py:5-15)."""
    import torch
    t = torch.linspace(1.0, eps, num_steps + 1)
    return [float((t[i] - t[i + 1]).item()) for i in range(num_steps)]


def _logits_np(model: Callable, ids: np.ndarray) -> np.ndarray:
    out = model(ids)["logits"]
    if hasattr(out, "detach"):
        out = out.detach().float().cpu().numpy()
    return np.asarray(out, dtype=np.float64)


def confidence(logits: np.ndarray, preds: np.ndarray, strategy: str) -> np.ndarray:
    """Per-position confidence of row-wise logits [L, V] (mask/pad already -inf)."""
    if strategy == "margin":
        srt = np.sort(logits, axis=-1)
        return srt[:, -1] - srt[:, -2]
    if strategy == "confidence":
        m = logits.max(axis=-1, keepdims=True)
        lse = m[:, 0] + np.log(np.exp(logits - m).sum(axis=-1))
        return logits[np.arange(logits.shape[0]), preds] - lse
    raise ValueError(f"strategy {strategy!r}")


def step_count(frac: float, target_len: int) -> int:
    """int(float32(frac * target_len)): the float32 product and truncation of
    diffusion_engine.py:65-66."""
    return int(np.float32(frac * target_len))


def select_step(logits: np.ndarray, masked: np.ndarray, want: int, strategy: str):
    """One unmasking step on target logits [B, T, V] whose mask and pad columns are
    already -inf (diffusion_engine.py:53-82): per row the argmax predictions, their
    confidences, and the min(want, masked count) still-masked positions of largest
    confidence (ties to the lower position).  Returns (preds [B, T] int64,
    conf [B, T] float64, chosen [B, T] bool)."""
    B, T, _ = logits.shape
    preds = np.zeros((B, T), dtype=np.int64)
    conf = np.zeros((B, T), dtype=np.float64)
    chosen = np.zeros((B, T), dtype=bool)
    for i in range(B):
        preds[i] = logits[i].argmax(axis=-1)
        conf[i] = confidence(logits[i], preds[i], strategy)
        cand = np.flatnonzero(masked[i])
        n = min(want, cand.size)
        if n == 0:
            continue
        # the n largest confidences among the masked positions
        chosen[i, cand[np.argsort(-conf[i, cand], kind="stable")[:n]]] = True
    return preds, conf, chosen


def diffusion_generate(model: Callable, prefix_ids: np.ndarray, target_len: int,
                       mask_token_id: int, pad_token_id: int, num_steps: int,
                       strategy: str = "confidence", stats: dict = None) -> np.ndarray:
    prefix_ids = np.asarray(prefix_ids, dtype=np.int64)
    B, P = prefix_ids.shape
    ids = np.concatenate(
        [prefix_ids, np.full((B, target_len), mask_token_id, dtype=np.int64)], axis=1)
    masked = np.ones((B, target_len), dtype=bool)
    forwards = 0
    for frac in linear_unmask_schedule(num_steps):
        logits = _logits_np(model, ids.copy())[:, P:]
        forwards += 1
        logits[:, :, mask_token_id] = -np.inf
        logits[:, :, pad_token_id] = -np.inf
        preds, _, chosen = select_step(logits, masked, step_count(frac, target_len), strategy)
        tgt = ids[:, P:]
        tgt[chosen] = preds[chosen]
        masked &= ~chosen
    if masked.any():
        logits = _logits_np(model, ids.copy())[:, P:]
        forwards += 1
        logits[:, :, mask_token_id] = -np.inf
        final = logits.argmax(axis=-1)
        tgt = ids[:, P:]
        tgt[masked] = final[masked]
    if stats is not None:
        stats["forwards"] = forwards
    return ids
