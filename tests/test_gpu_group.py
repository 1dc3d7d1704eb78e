"""GPU parity of the leaf-grouped step (ygg_run_grouped): streams that take the same expert at a (token, layer) are
updated together, large groups on int8 MFMA. Every leaf, state after every token, logit and digest must equal the
C oracle's exactly (the oracle is pinned to the reference kernel, cpu/ygg.cpp, in tests/test_oracle.py).

Cases: groups of every size (a router of 8 experts under 200 streams: several tiles per expert, MFMA tiles; 256
experts under a skewed router: groups of 1 to dozens), the configuration-4 router plan (D = 14: 4, 4, 3, 3), the
MFMA threshold at both ends (every tile on MFMA, none), a bad token that stops its stream, one stream, a carried
state, graph capture replayed with eager work between replays, and the full configuration-5 workload against the
per-stream kernel's digest and logit sums (itself checked against the oracle in test_gpu_fullsize.py).
"""
import numpy as np
import pytest

from oracle import oracle as O
from oracle.oracle import Oracle
from yggdrasil_amd import synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _load(path, mfma_min=None, monkeypatch=None):
    from yggdrasil_amd.inference import Yggdrasil
    if mfma_min is not None:
        monkeypatch.setenv("YGG_GROUP_MFMA_MIN", str(mfma_min))
    m = Yggdrasil.load(path)
    if mfma_min is not None:
        monkeypatch.delenv("YGG_GROUP_MFMA_MIN")
    return m


def _grouped(model, x, state=None):
    import torch
    r = model.run_grouped(x, state=state, leaves=True, states=True, digest=True)
    torch.cuda.synchronize()
    out = {k: v.cpu().numpy() for k, v in r.items()}
    out["digest"] = out["digest"].view(np.uint64)
    return out


def _same(got, ref, what):
    for k in ("leaves", "states", "logits", "state", "digest"):
        a, b = got[k], ref[k]
        assert a.shape == b.shape, (what, k, a.shape, b.shape)
        if not np.array_equal(a, b):
            bad = np.argwhere(a != b)
            raise AssertionError(f"{what}: {k}: {len(bad)} mismatches, first at {bad[:4].tolist()}: "
                                 f"gpu {a[tuple(bad[0])]} oracle {b[tuple(bad[0])]}")


def _model(model_dir, D, V, L, router, seed=5):
    path = model_dir / f"grp_{D}_{V}_{L}_{router}.bin"
    if not path.exists():
        synth.write_model(synth.ModelSpec(128, 16, D, V, L, router=router), seed, path)
    return path


CASES = [
    # D, V, L, router, B, T: 8 experts under 200 streams (tiles of 16, several per expert); 256 skewed experts;
    # the configuration-4 plan at a small vocabulary; one layer (the token layer only)
    (3, 27, 3, "gauss", 200, 6),
    (8, 256, 4, "skew", 300, 5),
    (14, 5, 4, "gauss", 96, 8),
    (14, 27, 3, "skew", 64, 4),
    (4, 256, 1, "gauss", 80, 5),
]


@pytest.mark.parametrize("case", CASES, ids=[f"D{c[0]}_V{c[1]}_L{c[2]}_{c[3]}" for c in CASES])
@pytest.mark.parametrize("mfma_min", [None, 1, 17])
def test_grouped_matches_oracle(model_dir, monkeypatch, case, mfma_min):
    """Leaves, states, logits, final state and digest of one grouped call equal the oracle's, with the default
    MFMA threshold, every tile on MFMA (1) and none (17: above the 16 streams of a tile)."""
    D, V, L, router, B, T = case
    path = _model(model_dir, D, V, L, router)
    x = synth.uniform_tokens(V, B, T, 9) if router == "gauss" else synth.zipf_bytes(B, T, 9) % V
    x = np.ascontiguousarray(x, np.int32)
    _say(f"grouped {case} mfma_min {mfma_min}")
    ref = Oracle(path).run(x, states=True, digest=True)
    model = _load(path, mfma_min, monkeypatch)
    assert model.info.grouped == 1
    got = _grouped(model, x)
    assert model.take_errors() == 0
    _same(got, ref, f"{case} mfma_min {mfma_min}")
    model.close()


def test_grouped_edges(model_dir):
    """One stream; a carried state and digest (two calls equal one); a bad token stops its stream there (error bit
    0; the other streams and the stream's earlier tokens exact); zero streams and zero tokens do nothing."""
    import torch
    path = _model(model_dir, 8, 256, 4, "skew")
    model = _load(path)
    orc = Oracle(path)
    x = np.ascontiguousarray(synth.zipf_bytes(40, 10, 3), np.int32)
    # one stream
    ref1 = orc.run(x[:1], states=True, digest=True)
    _same(_grouped(model, x[:1]), ref1, "one stream")
    # carried: tokens 0..3, then 4..9 from the state and digest after them
    ref = orc.run(x, states=True, digest=True)
    a = model.run_grouped(x[:, :4], leaves=True, states=True, digest=True)
    b = model.run_grouped(x[:, 4:], state=a["state"], leaves=True, states=True, digest=a["digest"])
    torch.cuda.synchronize()
    got = {k: np.concatenate([a[k].cpu().numpy(), b[k].cpu().numpy()], 1) for k in ("leaves", "states", "logits")}
    got["state"] = b["state"].cpu().numpy()
    got["digest"] = b["digest"].cpu().numpy().view(np.uint64)
    _same(got, ref, "carried")
    # a bad token at stream 7, token 5: the oracle's results for its first 5 tokens, the others whole
    xb = x.copy()
    xb[7, 5] = 256
    # (on the GPU: tokens given on the host are range-checked there first)
    r = model.run_grouped(torch.as_tensor(xb, device=model.device), leaves=True, states=True, digest=True)
    torch.cuda.synchronize()
    assert model.take_errors() & 1
    ok = np.arange(40) != 7
    lv, sv, lg = (r[k].cpu().numpy() for k in ("leaves", "states", "logits"))
    np.testing.assert_array_equal(lv[ok], ref["leaves"][ok])
    np.testing.assert_array_equal(sv[ok], ref["states"][ok])
    np.testing.assert_array_equal(lg[ok], ref["logits"][ok])
    np.testing.assert_array_equal(r["state"].cpu().numpy()[ok], ref["state"][ok])
    r7 = orc.run(x[7:8, :5], states=True, digest=True)
    np.testing.assert_array_equal(lv[7, :5], r7["leaves"][0])
    np.testing.assert_array_equal(sv[7, :5], r7["states"][0])
    np.testing.assert_array_equal(lg[7, :5], r7["logits"][0])
    np.testing.assert_array_equal(r["state"].cpu().numpy()[7], r7["state"][0])
    np.testing.assert_array_equal(r["digest"].cpu().numpy().view(np.uint64)[7], r7["digest"][0])
    # empty calls
    e = model.run_grouped(x[:0], leaves=True)
    assert e["logits"].shape == (0, 10, 256)
    z = model.run_grouped(x[:, :0], leaves=True)
    assert z["logits"].shape == (40, 0, 256)
    torch.cuda.synchronize()
    assert model.take_errors() == 0
    model.close()


@pytest.mark.parametrize("spec", [synth.ModelSpec(64, 16, 6, 27, 2), synth.ModelSpec(128, 16, 6, 27, 3, group=True),
                                  synth.ModelSpec(128, 16, 6, 27, 3, input_rank=16),
                                  synth.ModelSpec(128, 16, 15, 5, 2)],
                         ids=["d64", "group_scales", "factored", "depth15"])
def test_grouped_rejects_other_shapes(model_dir, spec):
    """Models outside the grouped step's shape (d_state 64, group scales, factored inputs, router depth 15) report
    YGG_ERR_LIMITS from both grouped entry points and run nothing."""
    import ctypes
    import torch
    from yggdrasil_amd import _lib
    path = model_dir / f"grp_reject_{spec.d_state}_{int(spec.group)}_{spec.input_rank}_{spec.router_depth}.bin"
    synth.write_model(spec, 1, path)
    model = _load(path)
    assert model.info.grouped == 0
    with pytest.raises(_lib.YggError) as e:
        model.run_grouped(np.zeros((2, 3), np.int32))
    assert _lib.ERRORS[e.value.code] == "limits"
    x = torch.zeros(2, 3, dtype=torch.int32, device=model.device)
    st = model.init_state(2)
    rc = _lib.lib().ygg_run_grouped_noalloc(model._h, ctypes.c_void_p(x.data_ptr()), 2, 3,
                                             ctypes.c_void_p(st.data_ptr()), None, None, None, None, None)
    assert _lib.ERRORS[rc] == "limits"
    model.close()


def test_grouped_many_streams(model_dir):
    """20 000 streams (the plan's streams-per-thread passes run three times; the workspace grows past an earlier
    call's) against the per-stream kernel on the same inputs: leaves, final state and digest equal."""
    import torch
    path = _model(model_dir, 3, 27, 3, "gauss")
    model = _load(path)
    small = model.run_grouped(np.ascontiguousarray(synth.uniform_tokens(27, 100, 2, 1), np.int32))
    x = torch.as_tensor(synth.uniform_tokens(27, 20000, 3, 2), device=model.device)
    a = model.run(x, logits=False, leaves=True, digest=True)
    b = model.run_grouped(x, logits=False, leaves=True, digest=True)
    torch.cuda.synchronize()
    del small
    for k in ("leaves", "state", "digest"):
        assert torch.equal(a[k], b[k]), k
    assert model.take_errors() == 0
    model.close()


def test_grouped_graph_replay(model_dir):
    """A grouped call captured in a hipGraph (after an eager call of as many streams, which sizes the workspace) and
    replayed three times, eager work and a sync between replays, every replay equal to the oracle."""
    import ctypes
    import torch
    from yggdrasil_amd import _lib
    path = _model(model_dir, 3, 27, 3, "gauss")
    B, T = 120, 4
    x = np.ascontiguousarray(synth.uniform_tokens(27, B, T, 4), np.int32)
    ref = Oracle(path).run(x, states=True, digest=True)
    model = _load(path)
    xt = torch.as_tensor(x, device=model.device)
    st = model.init_state(B)
    lg = torch.empty(B, T, 27, device=model.device)
    lv = torch.empty(B, T, 3, dtype=torch.int32, device=model.device)
    dg = torch.empty(B, dtype=torch.int64, device=model.device)
    L_ = _lib.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731

    def call(s):
        _lib.check(L_.ygg_run_grouped(model._h, p(xt), B, T, p(st), p(lg), p(lv), None, p(dg), s))

    call(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))      # sizes the workspace
    torch.cuda.synchronize()
    init = torch.tensor(np.array([O.DIGEST_INIT], np.uint64).view(np.int64), device=model.device)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    for i in range(3):
        st.zero_()
        lg.zero_()
        lv.fill_(-7)
        dg.copy_(init.expand(B))
        g.replay()
        _ = torch.randn(1000, device=model.device).sum()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(lg.cpu().numpy(), ref["logits"], err_msg=f"replay {i}")
        np.testing.assert_array_equal(lv.cpu().numpy(), ref["leaves"], err_msg=f"replay {i}")
        np.testing.assert_array_equal(st.cpu().numpy(), ref["state"], err_msg=f"replay {i}")
        np.testing.assert_array_equal(dg.cpu().numpy().view(np.uint64), ref["digest"], err_msg=f"replay {i}")
    assert model.take_errors() == 0
    model.close()


@pytest.mark.timeout(600)
def test_grouped_full_size_c5():
    """The full configuration-5 workload (8192 streams x 512 tokens, skewed router) in one grouped call: per-stream
    digest, logit bit sums and final state equal the C oracle's and the per-stream kernel's (ygg_run) on the same
    inputs."""
    import os
    import time
    import torch
    from pathlib import Path
    from yggdrasil_amd.inference import Yggdrasil
    w = synth.CONFIGS[5]
    cache = Path(os.environ.get("YGG_BENCH_DIR", "/tmp/ygg_bench"))
    cache.mkdir(parents=True, exist_ok=True)
    path = cache / f"{w.name}_seed{w.model_seed}.bin"
    if not path.exists():
        tmp = path.with_suffix(".tmp")
        synth.write_model(w.spec, w.model_seed, tmp)
        os.replace(tmp, path)
    x = w.make_tokens()
    B, T = x.shape
    model = Yggdrasil.load(path)
    xt = torch.as_tensor(x, device=model.device)

    def sums(r):
        lg = r["logits"]
        out = torch.empty(B, dtype=torch.int64, device=model.device)
        for b0 in range(0, B, 256):
            out[b0:b0 + 256] = (lg[b0:b0 + 256].view(torch.int32).to(torch.int64) & 0xFFFFFFFF).sum(dim=(1, 2))
        return out.cpu().numpy(), r["digest"].cpu().numpy(), r["state"].cpu().numpy()

    t0 = time.time()
    a = sums(model.run(xt, digest=True))
    torch.cuda.synchronize()
    _say(f"c5 per-stream kernel done in {time.time() - t0:.1f}s")
    torch.cuda.empty_cache()
    t0 = time.time()
    b = sums(model.run_grouped(xt, digest=True))
    torch.cuda.synchronize()
    _say(f"c5 grouped done in {time.time() - t0:.1f}s")
    assert model.take_errors() == 0
    for name, u, v in zip(("logit sums", "digest", "state"), a, b):
        bad = np.argwhere(u != v)
        assert bad.size == 0, f"{name} differs at {bad[:4].tolist()}"
    t0 = time.time()
    rdg, rls, rst = Oracle(path).run_sums(x)
    _say(f"c5 oracle done in {time.time() - t0:.1f}s")
    for name, u, v in zip(("logit sums", "digest", "state"), b, (rls, rdg, rst)):
        bad = np.argwhere(u.astype(np.uint64) != v.astype(np.uint64)) if name != "state" else np.argwhere(u != v)
        assert bad.size == 0, f"grouped {name} differs from the oracle at {bad[:4].tolist()}"
    model.close()
