"""Writes tests/golden/fixtures.npz: small seeded cases with the oracle's
outputs (projections, Q8_K, dequantised rows, top-k, GeGLU), so the GPU
path is checked against frozen vectors as well as against the live oracle.

Usage: python tests/golden/make_fixtures.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from heliopause_amd import synthetic as S  # noqa: E402
from oracle import oracle as O  # noqa: E402


def main() -> None:
    f = {}
    seed = S.derive(S.BASE_SEED, "fixtures")
    f["q4k_w"] = S.q4_k_blocks(S.derive(seed, 1), 13, 512)
    f["q4k_x"] = S.activations(S.derive(seed, 2), 3, 512)
    f["q4k_out"] = O.matmul(O.Q4_K, f["q4k_w"], f["q4k_x"], 13)
    f["q4k_deq"] = np.stack([O.dequantize(O.Q4_K, r, 512) for r in f["q4k_w"]])
    qs, d, bs = O.quantize_q8_k(f["q4k_x"])
    f["q4k_x_qs"], f["q4k_x_d"], f["q4k_x_bsums"] = qs, d, bs
    f["q6k_w"] = S.q6_k_blocks(S.derive(seed, 3), 7, 2560)
    f["q6k_x"] = S.activations(S.derive(seed, 4), 2, 2560)
    f["q6k_out"] = O.matmul(O.Q6_K, f["q6k_w"], f["q6k_x"], 7)
    f["q6k_deq"] = np.stack([O.dequantize(O.Q6_K, r, 2560) for r in f["q6k_w"][:2]])
    specs = [(O.Q4_K, 16), (O.Q4_K, 8), (O.Q6_K, 8)]
    ws = [(S.q4_k_blocks if t == O.Q4_K else S.q6_k_blocks)(S.derive(seed, 10 + i), r, 2560)
          for i, (t, r) in enumerate(specs)]
    x = S.activations(S.derive(seed, 5), 4, 2560)
    outs = O.matmul_multi([t for t, _ in specs], ws, x, [r for _, r in specs])
    for i, (w, o) in enumerate(zip(ws, outs)):
        f[f"multi_w{i}"], f[f"multi_out{i}"] = w, o
    f["multi_x"] = x
    rng = np.random.default_rng(7)
    logits = rng.integers(-20, 21, (2, 4096)).astype(np.float32) * 0.25
    logits[1, ::3] = -0.0
    f["topk_logits"] = logits
    ids, vals = zip(*[O.topk(r, 40) for r in logits])
    f["topk_ids"], f["topk_vals"] = np.stack(ids), np.stack(vals)
    g = (rng.standard_normal(4096) * 3).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    f["geglu_gate"], f["geglu_up"], f["geglu_out"] = g, u, O.geglu(g, u)
    out = Path(__file__).resolve().parent / "fixtures.npz"
    np.savez_compressed(out, **f)
    print(out, out.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
