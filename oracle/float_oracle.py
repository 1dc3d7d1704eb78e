"""TEST INFRASTRUCTURE ONLY: a float64 NumPy restatement of the float inference step, the checker of the float
kernel (csrc/ygg_float.hip). Only tests/ import this module.

It follows yggdrasil/inference.py:42-74 (route, update, step) and the calibration maxima of cpu/export.py:127-153:

    route:   node = 2 node + 1 + ([router_embed[x]; rms(h_below)] . W[node] + b[node] > 0), D times; leaf = node - E + 1
    update:  h = T_r[x] + U'_r (V' rms(h_below)) + A_r h_old
    readout: logits = output_bias + sum_l Q_l (P_r h)
    rms(h) = h / sqrt(mean(h^2) + 1e-6)

over FloatLayers of yggdrasil_amd.float_model (T_r[x] and A_r precomputed there).
"""
from __future__ import annotations

import numpy as np

RMS_EPS = 1e-6


def rms(h: np.ndarray) -> np.ndarray:
    return h / np.sqrt(np.mean(np.square(h), -1, keepdims=True) + RMS_EPS)


def route(layer, x: np.ndarray, below: np.ndarray) -> np.ndarray:
    """Leaf (B,) of tokens x (B,) given rms(h_below) (B, n) (yggdrasil/inference.py:42-51)."""
    f = layer.router_embed[x]
    if layer.routes_on_state:
        f = np.concatenate([f, below], -1)
    node = np.zeros(len(x), np.int64)
    for _ in range(layer.depth):
        s = np.einsum("bf,bf->b", f, layer.router_weight[node]) + layer.router_bias[node]
        node = 2 * node + 1 + (s > 0)
    return node - (2 ** layer.depth - 1)


def run(layers, output_bias, tokens: np.ndarray, state=None) -> dict:
    """tokens (B, T) -> dict(logits (B, T, C), leaves (B, T, L), state (B, L, n), stats (L, 3 + n/16 + R))."""
    x_all = np.asarray(tokens, np.int64)
    B, T = x_all.shape
    L, n = len(layers), layers[0].n
    R = layers[0].readout.shape[1]
    st = np.zeros((B, L, n)) if state is None else np.array(state, np.float64)
    C = len(output_bias)
    logits = np.empty((B, T, C))
    leaves = np.empty((B, T, L), np.int32)
    stats = np.zeros((L, 3 + n // 16 + R))
    for t in range(T):
        x = x_all[:, t]
        lg = np.broadcast_to(np.asarray(output_bias, np.float64), (B, C)).copy()
        below = None
        for i, p in enumerate(layers):
            r = x if i == 0 else route(p, x, below)
            h = p.table[x] if i == 0 else p.table[r, x]
            if i and p.layer_input_down is not None:
                zl = below @ p.layer_input_down.T
                stats[i, 1] = max(stats[i, 1], np.abs(zl).max())
                h = h + np.einsum("bkr,br->bk", p.layer_input_proj[r], zl)
            if p.transition is not None:
                a = p.transition[r]
                h = h + np.einsum("bgij,bgj->bgi", a, st[:, i].reshape(a.shape[:-1])).reshape(B, n)
            z = np.einsum("brk,bk->br", p.readout[r], h)
            st[:, i] = h
            below = rms(h)
            lg = lg + z @ p.unembed.T
            leaves[:, t, i] = r
            ah = np.abs(h)
            stats[i, 0] = max(stats[i, 0], ah.max())
            stats[i, 3:3 + n // 16] = np.maximum(stats[i, 3:3 + n // 16], ah.reshape(B, n // 16, 16).max((0, 2)))
            az = np.abs(z).max(0)
            stats[i, 2] = max(stats[i, 2], az.max())
            stats[i, 3 + n // 16:] = np.maximum(stats[i, 3 + n // 16:], az)
        logits[:, t] = lg
    return dict(logits=logits, leaves=leaves, state=st, stats=stats)
