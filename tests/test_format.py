"""YGG1 files written by yggdrasil_amd.fmt / synth: header LIMITS, array table, packers, deterministic generation.

The packed layouts are pinned by the reference kernel reading these files (tests/test_oracle.py) and by the
reference's int_forward on logical arrays (configuration 3 in tests/golden/golden.json); here each packer is
checked against the index formula of the layout it documents, the header against LIMITS (cpu/export.py:353-379), and
the chunk-streamed writer of large models against the in-memory writer.
"""
import hashlib

import numpy as np
import pytest

from yggdrasil_amd import fmt, synth


def test_header_limits_name_the_field():
    layers = synth.random_layers(synth.KERNEL_CASES[3], 1)
    for field, value in (("d_state", 80), ("block_size", 4), ("readout_rank", 12)):
        bad = [fmt.QuantLayer(**{**q.__dict__}) for q in layers]
        for q in bad:
            if field == "d_state":
                q.n = value
            if field == "block_size":
                q.block = value
        if field == "readout_rank":
            bad[0].readout = np.zeros((5, 12, 64), np.int8)
        with pytest.raises(ValueError, match=field):
            fmt.header(bad, 5)
    with pytest.raises(ValueError, match="vocab"):
        fmt.header(layers, 300)


def test_container_round_trip(tmp_path):
    spec = synth.KERNEL_CASES[13]       # factored + group scales
    path = tmp_path / "m.bin"
    synth.write_model(spec, 2, path)
    mf = fmt.read(path)
    h = mf.header
    assert (h["n_layers"], h["d_state"], h["block_size"], h["vocab"], h["router_depth"], h["readout_rank"],
            h["layer_input_rank"], h["input_rank"], h["shift"]) == (3, 128, 16, 256, 7, 16, 32, 32, 14)
    VP = 256
    assert mf.array("head_b", np.float32).shape == (VP,)
    for l in range(3):
        meta = mf.array(f"l{l}_meta", np.int32)
        assert len(meta) == (8 if l else 5)
        assert meta[0] % 64 == 0
        rec = mf.arrays[f"l{l}_rec"]
        E = 256 if l == 0 else 128
        assert rec.size == E * meta[0]
        assert mf.arrays[f"l{l}_Q"].size == 16 * VP
    assert mf.arrays["l1_thr"].size == 4 * 256 * 128
    assert mf.arrays["l1_w"].size == 128 * 128
    assert set(("l1_vt", "l1_mT", "l1_r2b", "l1_mulv", "l1_mzl", "l0_sqv")) <= set(mf.arrays)
    # offsets are 64-aligned
    data = np.fromfile(path, np.uint8)
    base = fmt.round_up(fmt.HEADER_STRUCT.size + h["n_arrays"] * fmt.ENTRY_STRUCT.size, 64)
    for a in fmt.parse(data).arrays.values():       # views of `data`: offsets from its start
        assert (a.__array_interface__["data"][0] - data.__array_interface__["data"][0] - base) % 64 == 0


def test_pack_transition_index():
    rng = np.random.default_rng(0)
    for n, b in ((64, 8), (96, 16), (128, 16)):
        A = rng.integers(-2 ** 15, 2 ** 15, (3, n // b, b, b)).astype(np.int16)
        p = fmt.pack_transition(A).view("<i2")
        for e in range(3):
            for i in range(0, n, 7):
                for j in range(b):
                    g, rr = i // 16, i % 16
                    o = ((g * (b // 2) + j // 2) * 16 + rr) * 2 + (j & 1)
                    assert p[e, o] == A[e, i // b, i % b, j]


def test_pack_proj_readout_unembed_index():
    rng = np.random.default_rng(1)
    n = 96
    U = rng.integers(-127, 128, (2, n, 20)).astype(np.int8)
    p = fmt.pack_proj(U)
    for i in range(0, n, 5):
        for k in range(20):
            assert int(p[1, ((k // 4) * n + i) * 4 + k % 4]) - 128 == U[1, i, k]
    for R in (8, 16, 32):
        P = rng.integers(-127, 128, (2, R, n)).astype(np.int8)
        p = fmt.pack_readout(P)
        for j in range(R):
            for i in range(0, n, 3):
                if R == 8:
                    o = ((i // 8) * 16 + 2 * j + (i % 8) // 4) * 4 + i % 4
                else:
                    o = (((j // 16) * (n // 4) + i // 4) * 16 + j % 16) * 4 + i % 4
                assert int(p[1, o]) - 128 == P[1, j, i]
    Q = rng.integers(-127, 128, (27, 8)).astype(np.int8)
    p = fmt.pack_unembed(Q, 32)
    flat = p.reshape(-1)
    for c in range(32):
        for j in range(8):
            v = int(flat[((j // 4) * 32 + c) * 4 + j % 4]) - 128
            assert v == (Q[c, j] if c < 27 else 0)


@pytest.mark.parametrize("group", [False, True], ids=["tensor", "group"])
def test_generation_is_deterministic_and_streaming_matches(tmp_path, monkeypatch, group):
    # 2048 experts: two chunks per routed layer; group scales add the per-expert readout scale array
    spec = synth.ModelSpec(64, 16, 11, 27, 3, router="skew", group=group)
    a, b = tmp_path / "a.bin", tmp_path / "b.bin"
    synth.write_model(spec, 5, a)
    # force the chunk-streamed path used for large models
    real = synth._experts
    calls = []

    def spy(*args, **kw):
        calls.append(args[3:5])
        return real(*args, **kw)
    monkeypatch.setattr(synth, "_experts", spy)
    monkeypatch.setattr(synth, "_small_limit", 0)
    synth.write_model(spec, 5, b)
    assert any(j1 - j0 == synth.CHUNK for j0, j1 in calls), "streamed path not taken"
    ha = hashlib.sha256(a.read_bytes()).hexdigest()
    hb = hashlib.sha256(b.read_bytes()).hexdigest()
    assert ha == hb


def test_token_generators():
    z = synth.zipf_bytes(64, 512, 1)
    counts = np.bincount(z.ravel(), minlength=256)
    assert counts[0] > counts[1] > counts[10] > counts[100]
    d = synth.dna_tokens(64, 512, 2)
    assert d.max() == 4 and 0 < np.mean(d == 4) < 0.005
    u = synth.uniform_tokens(256, 4, 4, 0)
    assert u.dtype == np.int32 and u.shape == (4, 4)
