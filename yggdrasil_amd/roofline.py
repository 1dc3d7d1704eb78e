"""Algorithmic (compulsory) HBM bytes of the int8 step, computed from the leaves a run actually took.

Per batched step (one token for each of B streams), the bytes no implementation can avoid reading are the distinct
weights that step touches, plus the per-stream inputs and outputs:

    sum over routed layers l of
        distinct leaves r        x (2 n b + n R2 + R n)     transition A16, layer-input U', readout P
                                   (factored: + k n + 2 n + 4, the input projection U_r, bias c_r and scale)
        distinct (r, x)          x 2 n                      table row T_r[x] (table storage)
        distinct tokens x        x k                        token code v[x] (factored storage, rank k)
        distinct router nodes    x n                        router rows on the paths taken
        distinct (x, node)       x 4                        thresholds thr[x][node]
    + distinct tokens x          x (2 n b + R n + 2 n)      token layer: A16, P and its own table row
    + B x (4 + 4 V)                                         token in, logits out

With group scales every expert also carries its R readout row scales (4 R bytes, per distinct leaf and per distinct
token for the token layer); the per-class and per-coordinate scale vectors are read once per launch and left out.

and once per launch the int8 state of every stream in and out, 2 B L n. A T-token launch sums the T steps; the
per-token figure is measured on an evenly spaced sample of the steps (all of them when T <= sample) and multiplied by
the B T tokens of the launch. The per-stream figure (no deduplication across streams) is reported beside it.
"""
from __future__ import annotations

import numpy as np


def step_bytes(leaves: np.ndarray, tokens: np.ndarray, n: int, b: int, R: int, R2: int, V: int, D: int,
               factored_rank: int = 0, sample: int = 64, group: bool = False) -> dict:
    """leaves (B, T, L) int (layer 0: the token), tokens (B, T) -> dict(compulsory=, per_stream=) bytes of the whole
    T-token launch, the per-launch state bytes in 'state' and the per-token figures."""
    B, T, L = leaves.shape
    E = 1 << D
    leaf_w = 2 * n * b + n * R2 + R * n + ((factored_rank * n + 2 * n + 4) if factored_rank else 0)
    row_w = 0 if factored_rank else 2 * n
    tok_w = 2 * n * b + R * n + 2 * n
    if group:
        leaf_w += 4 * R
        tok_w += 4 * R
    io = B * (4 + 4 * V)
    comp = 0
    per = 0
    x_all = tokens.astype(np.int64)
    steps = np.unique(np.linspace(0, T - 1, min(T, sample)).round().astype(np.int64))
    for t in steps:
        x = x_all[:, t]
        comp += np.unique(x).size * tok_w + io
        per += B * tok_w + io
        for l in range(1, L):
            r = leaves[:, t, l].astype(np.int64)
            comp += np.unique(r).size * leaf_w
            comp += np.unique(r * V + x).size * row_w + np.unique(x).size * factored_rank
            # the path of leaf r: node at depth d is (r + E) >> (D - d), d = 0 .. D-1
            d = np.arange(D, dtype=np.int64)
            nodes = (r[:, None] + E) >> (D - d)[None, :]
            comp += np.unique(nodes).size * n
            comp += np.unique(x[:, None] * E + nodes).size * 4
            per += B * (leaf_w + row_w + factored_rank + D * (n + 4))
    scale = T / len(steps)
    state = 2 * B * L * n
    comp, per = comp * scale + state, per * scale + state
    return dict(compulsory=int(comp), per_stream=int(per), state=int(state), steps_sampled=int(len(steps)),
                per_token_compulsory=comp / (B * T), per_token_per_stream=per / (B * T))
