"""The algorithmic (compulsory) byte count behind bench.py's roofline (yggdrasil_amd.roofline.step_bytes), against
counts by hand: one stream, two streams sharing their leaf or on neighbouring leaves, factored storage and group
scales."""
import numpy as np

from yggdrasil_amd.roofline import step_bytes

n, b, R, R2, V, D = 128, 16, 8, 16, 256, 14
LEAF = 2 * n * b + n * R2 + R * n            # A16 + U' + P of a routed leaf
ROW = 2 * n                                   # its table row T_r[x]
TOK = 2 * n * b + R * n + 2 * n               # token layer: A16, P, its table row
IO = 4 + 4 * V                                # token in, logits out
STATE = 2 * 2 * n                             # int8 state of 2 layers, in and out, per stream


def _bytes(tokens, leaves, **kw):
    """One token per stream, 2 layers: the token layer and one routed layer with the given leaves."""
    x = np.asarray(tokens).reshape(-1, 1)
    lv = np.stack([x[:, 0], np.asarray(leaves)], 1)[:, None, :]
    return step_bytes(lv, x, n, b, R, R2, V, D, **kw)


def test_single_stream_closed_form():
    r = _bytes([7], [5])
    want = TOK + IO + LEAF + ROW + D * n + D * 4 + STATE     # D router rows and thresholds on the path
    assert r["compulsory"] == want and r["per_stream"] == want


def test_shared_and_neighbouring_leaves():
    one = _bytes([7], [5])["compulsory"]
    same = _bytes([7, 7], [5, 5])
    # identical streams read the same weights once; only input, output and state are per stream
    assert same["compulsory"] == one + IO + STATE and same["per_stream"] == 2 * one
    # leaves 5 and 6 share the path down to depth D - 2 (D - 1 nodes) and differ at depth D - 1; tokens 7 and 9
    # differ, so every threshold and table row is the stream's own
    other = _bytes([7, 9], [5, 6])
    want = 2 * (TOK + IO + LEAF + ROW + D * 4 + STATE) + (D + 1) * n
    assert other["compulsory"] == want
    # leaves 4 and 5 are siblings: the same D nodes
    sib = _bytes([7, 9], [4, 5])
    assert sib["compulsory"] == want - n


def test_factored_storage():
    k = 64
    fac = k * n + 2 * n + 4                   # U_r, c_r and the scale s_r, once per leaf
    t = _bytes([7, 9], [5, 5], factored_rank=k)
    # one leaf, no table rows, a token code v[x] per token
    want = 2 * (TOK + IO + D * 4 + STATE) + LEAF + fac + D * n + 2 * k
    assert t["compulsory"] == want
    assert t["per_stream"] == 2 * (TOK + IO + LEAF + fac + k + D * (n + 4) + STATE)


def test_group_scales():
    # the R readout row scales (f32) of every distinct expert: the routed leaf and each distinct token's expert
    t = _bytes([7, 9], [5, 5], group=True)
    base = _bytes([7, 9], [5, 5])
    assert t["compulsory"] == base["compulsory"] + 4 * R * 3
    assert t["per_stream"] == base["per_stream"] + 2 * 4 * R * 2
