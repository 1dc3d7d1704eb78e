"""The float model and the int8 export on the CPU: checkpoint reading, the precomputed transitions, the float64
restatement of the float step (oracle/float_oracle.py, the checker of the float kernel) on closed forms, and
yggdrasil_amd.export.quantize against the reference's own quantize (tests/golden/quant_golden.npz, written by
tests/golden/make_quant_golden.py from /root/reference/cpu/export.py)."""
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import float_oracle as FO
from yggdrasil_amd import float_model as FM
from yggdrasil_amd.export import LayerStats, quantize, stats_from_array

GOLDEN = Path(__file__).resolve().parent / "golden" / "quant_golden.npz"


@pytest.fixture(scope="module")
def small(tmp_path_factory):
    spec = FM.FloatSpec(d_state=64, block_size=16, router_depth=4, vocab=24, n_layers=3)
    p = tmp_path_factory.mktemp("f") / "m.npz"
    FM.random_checkpoint(spec, 3, p)
    return spec, p


def test_read_new_and_old_keys(small, tmp_path):
    spec, p = small
    layers, ob = FM.read(p)
    assert len(layers) == spec.n_layers and ob.shape == (spec.vocab,)
    assert layers[1]["router_weight"].shape == (2 ** spec.router_depth - 1, spec.router_token_dim + spec.d_state)
    # the released checkpoints' names (root/branches/u_in/...) read the same
    old = {v: k for k, v in FM.KEY_ALIASES.items()}
    with np.load(p) as z:
        arrs = {"/".join(old.get(part, part) for part in k.split("/")): z[k] for k in z.files}
    q = tmp_path / "old.npz"
    np.savez(q, **arrs)
    l2, ob2 = FM.read(q)
    np.testing.assert_array_equal(ob, ob2)
    for a, b in zip(layers, l2):
        assert set(a) == set(b)
        for k in a:
            np.testing.assert_array_equal(a[k], b[k])


def test_read_rejects(small, tmp_path):
    spec, p = small
    with np.load(p) as z:
        arrs = {k: z[k] for k in z.files}
    bad = dict(arrs, **{"token_layer/mystery": np.zeros(3, np.float32)})
    np.savez(tmp_path / "b1.npz", **bad)
    with pytest.raises(NotImplementedError, match="mystery"):
        FM.read(tmp_path / "b1.npz")
    bad = dict(arrs)
    bad["token_layer/readout"] = bad["token_layer/readout"][:1]
    np.savez(tmp_path / "b2.npz", **bad)
    with pytest.raises(NotImplementedError, match="one matrix per expert"):
        FM.read(tmp_path / "b2.npz")


def test_transitions_closed_forms():
    rng = np.random.default_rng(0)
    E, g, b = 3, 2, 4
    dec = rng.uniform(-1.5, 1.5, (E, g * b))
    # zero generator: A = diag(clip(decay))
    A = FM.transitions(np.zeros((E, g, b, b)), dec)
    want = np.zeros((E, g, b, b))
    for e in range(E):
        for j in range(g):
            want[e, j] = np.diag(np.clip(dec[e, j * b:(j + 1) * b], -1, 1))
    np.testing.assert_allclose(A, want, atol=1e-15)
    # any generator: the rotation part is orthogonal, and only the antisymmetric part of G matters
    G = rng.normal(0, 1, (E, g, b, b))
    A = FM.transitions(G, np.ones((E, g * b)))
    np.testing.assert_allclose(A @ np.swapaxes(A, -1, -2), np.broadcast_to(np.eye(b), A.shape), atol=1e-12)
    sym = rng.normal(0, 1, (E, g, b, b))
    np.testing.assert_allclose(FM.transitions(G + sym + np.swapaxes(sym, -1, -2), np.ones((E, g * b))), A, atol=1e-12)
    # b = 2: expm of [[0, -t], [t, 0]] is the rotation by t
    t = 0.3
    G2 = np.array([[[[0.0, -t], [t, 0.0]]]])
    np.testing.assert_allclose(FM.transitions(G2, np.ones((1, 2)))[0, 0],
                               [[math.cos(t), -math.sin(t)], [math.sin(t), math.cos(t)]], atol=1e-14)


def _layers(small):
    spec, p = small
    raw, ob = FM.read(p)
    return FM.float_layers(raw), ob, spec


def test_oracle_without_memory_is_a_lookup(small):
    """Decay 0 and no layer input: the state is the table row alone and the logits are bias + sum Q P T_r[x]."""
    layers, ob, spec = _layers(small)
    for fl in layers:
        fl.transition = np.zeros_like(fl.transition)
        fl.layer_input_down = fl.layer_input_proj = None
    x = np.random.default_rng(1).integers(0, spec.vocab, (3, 7))
    r = FO.run(layers, ob, x)
    for s in range(3):
        for t in range(7):
            lg = ob.astype(np.float64).copy()
            for i, fl in enumerate(layers):
                leaf = r["leaves"][s, t, i]
                h = fl.table[x[s, t]] if i == 0 else fl.table[leaf, x[s, t]]
                lg = lg + fl.unembed @ (fl.readout[leaf] @ h)
            np.testing.assert_allclose(r["logits"][s, t], lg, rtol=1e-12, atol=1e-12)


def test_oracle_forced_routes(small):
    """Router weights 0 and biases +-1 force every path: node j goes right iff its bias is positive."""
    layers, ob, spec = _layers(small)
    D = spec.router_depth
    rng = np.random.default_rng(2)
    for fl in layers[1:]:
        fl.router_weight = np.zeros_like(fl.router_weight)
        fl.router_bias = rng.choice([-1.0, 1.0], fl.router_bias.shape)
    x = rng.integers(0, spec.vocab, (4, 5))
    r = FO.run(layers, ob, x)
    for i, fl in enumerate(layers[1:], 1):
        node = 0
        for _ in range(D):
            node = 2 * node + 1 + int(fl.router_bias[node] > 0)
        assert (r["leaves"][:, :, i] == node - (2 ** D - 1)).all()


def test_oracle_rms_and_carry(small):
    layers, ob, spec = _layers(small)
    h = np.random.default_rng(3).normal(0, 2, (5, 64))
    y = FO.rms(h)
    np.testing.assert_allclose(np.mean(y ** 2, -1), np.mean(h ** 2, -1) / (np.mean(h ** 2, -1) + 1e-6), rtol=1e-12)
    x = np.random.default_rng(4).integers(0, spec.vocab, (2, 12))
    whole = FO.run(layers, ob, x)
    a = FO.run(layers, ob, x[:, :5])
    b = FO.run(layers, ob, x[:, 5:], state=a["state"])
    np.testing.assert_allclose(np.concatenate([a["logits"], b["logits"]], 1), whole["logits"], rtol=1e-13, atol=1e-13)


def _forced(layers, rng):
    """Router weights 0 and biases +-1: every leaf is fixed whatever the state (see test_oracle_forced_routes)."""
    for fl in layers[1:]:
        fl.router_weight = np.zeros_like(fl.router_weight)
        fl.router_bias = rng.choice([-1.0, 1.0], fl.router_bias.shape)


def test_oracle_identity_transition_accumulates(small):
    """A_r = I and no layer input: every layer's state is the running sum of the table rows it took,
    h_t = sum_{s <= t} T_{r_s}[x_s]."""
    layers, ob, spec = _layers(small)
    rng = np.random.default_rng(5)
    _forced(layers, rng)
    for fl in layers:
        g, b = fl.transition.shape[1], fl.transition.shape[2]
        fl.transition = np.broadcast_to(np.eye(b), fl.transition.shape).copy()
        fl.layer_input_down = fl.layer_input_proj = None
    x = rng.integers(0, spec.vocab, (3, 9))
    r = FO.run(layers, ob, x)
    for i, fl in enumerate(layers):
        acc = np.zeros((3, spec.d_state))
        for t in range(9):
            rows = fl.table[x[:, t]] if i == 0 else fl.table[r["leaves"][:, t, i], x[:, t]]
            acc = acc + rows
        np.testing.assert_allclose(r["state"][:, i], acc, rtol=1e-12, atol=1e-12)


def test_oracle_transition_orientation(small):
    """One nonzero entry A[block g][row i][column j] = a and no layer input: coordinate g b + i takes a times the
    previous value of coordinate g b + j, every other coordinate is its table row alone; a transposed A or a wrong
    block offset moves the term to another coordinate."""
    layers, ob, spec = _layers(small)
    rng = np.random.default_rng(6)
    _forced(layers, rng)
    b = layers[0].transition.shape[-1]
    g, i, j, a = 1, 2, 5, 0.75
    for fl in layers:
        A = np.zeros_like(fl.transition)
        A[:, g, i, j] = a
        fl.transition = A
        fl.layer_input_down = fl.layer_input_proj = None
    x = rng.integers(0, spec.vocab, (4, 6))
    r = FO.run(layers, ob, x)
    for l, fl in enumerate(layers):
        prev = np.zeros((4, spec.d_state))
        for t in range(6):
            row = fl.table[x[:, t]] if l == 0 else fl.table[r["leaves"][:, t, l], x[:, t]]
            want = row.copy()
            want[:, g * b + i] += a * prev[:, g * b + j]
            got = FO.run(layers, ob, x[:, :t + 1])["state"][:, l]
            np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
            prev = want


def test_oracle_rank_one_layer_input(small):
    """V' = e_0 e_k^T (only row 0, column k) and U'_r = c e_m e_0^T, no transitions: a routed layer's state is its
    table row plus c rms(h_below)[k] at coordinate m, with h_below the layer below after the same token."""
    layers, ob, spec = _layers(small)
    rng = np.random.default_rng(7)
    _forced(layers, rng)
    k, m, c = 9, 33, -1.25
    for fl in layers:
        fl.transition = np.zeros_like(fl.transition)
        if fl.layer_input_down is not None:
            Vd = np.zeros_like(fl.layer_input_down)
            Vd[0, k] = 1.0
            Up = np.zeros_like(fl.layer_input_proj)
            Up[:, m, 0] = c
            fl.layer_input_down, fl.layer_input_proj = Vd, Up
    assert layers[1].layer_input_down is not None
    x = rng.integers(0, spec.vocab, (5, 4))
    r = FO.run(layers, ob, x)
    st = FO.run(layers, ob, x[:, :3])["state"]
    for l in range(1, spec.n_layers):
        below = st[:, l - 1]
        mean_sq = (below ** 2).mean(-1)
        want = layers[l].table[r["leaves"][:, 2, l], x[:, 2]].copy()
        want[:, m] += c * below[:, k] / np.sqrt(mean_sq + 1e-6)
        np.testing.assert_allclose(st[:, l], want, rtol=1e-12, atol=1e-12)


def test_oracle_readout_orientation(small):
    """P_r = e_j e_k^T (readout row j reads coordinate k) and Q = e_c e_j^T (class c reads readout row j) in every
    layer: the logits are the output bias plus, at class c only, the sum over layers of h_l[k]."""
    layers, ob, spec = _layers(small)
    rng = np.random.default_rng(8)
    _forced(layers, rng)
    j, k, c = 3, 17, 11
    for fl in layers:
        P = np.zeros_like(fl.readout)
        P[:, j, k] = 1.0
        Q = np.zeros_like(fl.unembed)
        Q[c, j] = 1.0
        fl.readout, fl.unembed = P, Q
    x = rng.integers(0, spec.vocab, (3, 5))
    r = FO.run(layers, ob, x)
    want = np.broadcast_to(ob.astype(np.float64), (3, len(ob))).copy()
    want[:, c] += r["state"][:, :, k].sum(-1)
    np.testing.assert_allclose(r["logits"][:, -1], want, rtol=1e-12, atol=1e-12)


# ----------------------------------------------------------------------------------------------- quantisation
def _golden_setup():
    import importlib.util
    spec = importlib.util.spec_from_file_location("mqg", Path(__file__).resolve().parent / "golden" /
                                                  "make_quant_golden.py")
    mqg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mqg)
    return mqg


def test_quantize_matches_reference(tmp_path):
    mqg = _golden_setup()
    z = np.load(GOLDEN, allow_pickle=False)
    layers, ob = mqg.model(tmp_path)
    assert mqg.layers_digest(layers) == str(z["layers_sha256"]), "synthetic float model generator drifted"
    stats = stats_from_array(z["stats"], mqg.SPEC.d_state)
    shared = {k: z[k] for k in z.files if k.startswith(mqg.SETTINGS[0][0] + "/") and k.split("/")[-1] in mqg.SHARED}
    checked = 0
    for name, hm, group, fac in mqg.SETTINGS:
        got = mqg.flatten(quantize(layers, stats, hm, group, fac), name, True)
        for k, v in got.items():
            key = k if k in z.files else mqg.SETTINGS[0][0] + k[len(name):]
            want = z[key] if key in z.files else shared[key]
            v = np.asarray(v)
            assert v.shape == want.shape and (v.dtype == want.dtype or v.dtype.kind == want.dtype.kind == "i"), k
            np.testing.assert_array_equal(v, want, err_msg=k)       # integer values, and float32 scales bit for bit
            checked += 1
        assert {k for k in z.files if k.startswith(name + "/")} <= set(got), name
    assert checked > 90


def test_quantize_plants_fail():
    """A wrong state scale or a dropped folded token part changes the quantised arrays (the check is sharp)."""
    mqg = _golden_setup()
    import tempfile
    with tempfile.TemporaryDirectory() as tmp:
        layers, ob = mqg.model(Path(tmp))
    z = np.load(GOLDEN, allow_pickle=False)
    stats = stats_from_array(z["stats"], mqg.SPEC.d_state)
    bad = [LayerStats(s.state_max * 1.001, s.layer_input_max, s.readout_max, s.state_group_max, s.readout_row_max)
           for s in stats]
    q = quantize(layers, bad, 1.0)
    assert not np.array_equal(q[1].table, z["tensor_1.0/1/table"])


def test_windows_pair_each_token_with_the_next():
    from yggdrasil_amd.export import windows
    ids = np.arange(23)
    x, y = windows(ids, 5, 10)
    assert x.shape == y.shape == (4, 5)                     # (23 - 1) // 5 windows
    np.testing.assert_array_equal(x.ravel(), np.arange(20))
    np.testing.assert_array_equal(y.ravel(), np.arange(1, 21))
    x, y = windows(ids, 5, 2)
    assert x.shape == (2, 5) and y[-1, -1] == 10


def test_export_calibrates_on_inputs_and_scores_targets(small, tmp_path, monkeypatch):
    """export() takes the calibration maxima over the input windows only and compares its candidates by the bits of
    the targets given the inputs (the reference: calibrate(cx), bpc(int_forward(cx), cy), cpu/export.py:554-561);
    without targets, (S, T + 1) windows split into inputs [:, :-1] and targets [:, 1:]."""
    from yggdrasil_amd import export as X
    spec, p = small
    seen = {"calib": [], "score": []}

    class NoKernel:
        def __init__(self, *a, **k):
            pass

        def close(self):
            pass

    def fake_calibrate(model, x):
        seen["calib"].append(np.array(x))
        return [LayerStats(1.0, 1.0, 1.0, np.ones(spec.d_state // 16), np.ones(8)) for _ in range(spec.n_layers)]

    def fake_bits(q, ob, x, y, F, K):
        seen["score"].append((np.array(x), np.array(y)))
        return 1.0

    import torch
    monkeypatch.setattr(X, "FloatYggdrasil", NoKernel)
    monkeypatch.setattr(X, "calibrate", fake_calibrate)
    monkeypatch.setattr(X, "int8_bits", fake_bits)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a: None)
    rng = np.random.default_rng(0)
    w = rng.integers(0, spec.vocab, (6, 9))
    X.export(p, tmp_path / "a.bin", w, hmargin=1.0, state_scale="tensor")
    np.testing.assert_array_equal(seen["calib"][0], w[:, :-1])
    np.testing.assert_array_equal(seen["score"][0][0], w[:, :-1])
    np.testing.assert_array_equal(seen["score"][0][1], w[:, 1:])
    x, y = X.windows(rng.integers(0, spec.vocab, 100), 8, 4)
    X.export(p, tmp_path / "b.bin", x, y, hmargin=1.0, state_scale="tensor")
    np.testing.assert_array_equal(seen["calib"][1], x)
    np.testing.assert_array_equal(seen["score"][1][1], y)
    with pytest.raises(ValueError):
        X.export(p, tmp_path / "c.bin", x, y[:, :-1])
