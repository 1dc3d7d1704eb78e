"""Writes tests/golden/softmax_golden.npz: rows of logits and what the reference's own softmax() (cpu/ygg.cpp:59-72)
returns for them, from the reference built here (oracle/_ref/ygg_softmax, `make -C oracle ref`).

    python tests/golden/make_softmax_golden.py

Rows for V in {5, 27, 256} (the benchmark vocabularies) and 17 (a partial last 16-lane vector): Gaussian logits at
spreads 0.1 to 300 (the widest clamp exp's argument at -87 and give subnormal terms), equal logits, one dominant
class.
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as O  # noqa: E402


def rows(V: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    parts = [(rng.standard_normal((8, V)) * s).astype(np.float32) for s in (0.1, 1.0, 5.0, 30.0, 300.0)]
    ties = np.zeros((2, V), np.float32)
    ties[1] = np.float32(-3.25)
    dom = np.full((2, V), -1000.0, np.float32)
    dom[:, 0] = 0.0
    dom[1, V - 1] = 7.0
    return np.concatenate(parts + [ties, dom])


def main():
    if not O.have_ref_softmax():
        raise SystemExit("oracle/_ref/ygg_softmax not built (make -C oracle ref)")
    out = {}
    for V, seed in ((5, 1), (17, 2), (27, 3), (256, 4)):
        lg = rows(V, seed)
        p, s = O.ref_softmax(lg)
        out[f"logits_{V}"], out[f"probs_{V}"], out[f"lse_{V}"] = lg, p, s
    np.savez_compressed(ROOT / "tests" / "golden" / "softmax_golden.npz", **out)
    print({k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
