"""Write the golden fixtures for the config-1 shape (2,048 tokens, d 768, F 3072,
E 16, top-2): one with fp32 activations and one with bf16.

    python tests/golden/make_golden.py

Each .npz holds sha256 digests of the generated inputs (pinning the synthetic
generator), the routing outputs of the oracle (topk_idx, counts, offsets, perm,
inv_pos — the bit-exact contract), its gates, and for 8 sampled tokens the
oracle's fp32 output rows plus every token's output L2 norm (bf16-storage mode,
the kernels' contract).  The reference (GeneT5) has no MoE and no tests, so these
vectors come from this build's oracle; they pin it against later change.
"""
import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402
from genet5_amd import synth  # noqa: E402

ROWS = np.array([0, 1, 17, 511, 1024, 1500, 2046, 2047])


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def make(dtype: str) -> dict:
    inp = synth.make_layer(2048, seed=0, dtype=dtype)
    ref = oracle.moe_forward(inp.x, inp.w_router, inp.w_gate, inp.w_up, inp.w_down, 2,
                             storage="bf16")
    return dict(
        sha_x=digest(inp.x), sha_w_router=digest(inp.w_router), sha_w_gate=digest(inp.w_gate),
        sha_w_up=digest(inp.w_up), sha_w_down=digest(inp.w_down),
        topk_idx=ref["topk_idx"].astype(np.int8), topk_w=ref["topk_w"],
        counts=ref["counts"], offsets=ref["offsets"],
        perm=ref["perm"].astype(np.int16), inv_pos=ref["inv_pos"].astype(np.int16),
        rows=ROWS, y_rows=ref["y"][ROWS].astype(np.float32),
        y_row_norms=np.linalg.norm(ref["y"].astype(np.float64), axis=1).astype(np.float32),
    )


def main():
    for dtype in ("f32", "bf16"):
        path = HERE / f"cfg1_{dtype}_seed0.npz"
        np.savez_compressed(path, **make(dtype))
        print(path, path.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
