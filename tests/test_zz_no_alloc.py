"""ygg_run_grouped_noalloc (the grouped step on a static device workspace, for callers that cannot allocate) against
ygg_run_grouped through the C-ABI, bit-exact: two calls in a row, the second with fewer streams and tokens (the
static workspace keeps the first call's contents), a call of configuration 5's stream count, a replay of a captured
call, and a call beyond the workspace's limit, which is refused with YGG_ERR_LIMITS.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from yggdrasil_amd import synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


class _Call:
    """Outputs of one C-ABI call of either entry point on fresh buffers."""

    def __init__(self, model, x, entry):
        import torch
        from yggdrasil_amd import _lib
        B, T = x.shape
        info = model.info
        dev = model.device
        self.x = torch.as_tensor(x, device=dev).contiguous()
        self.state = model.init_state(B)
        self.logits = torch.full((B, T, info.vocab), -1.0, device=dev)
        self.leaves = torch.full((B, T, info.n_layers), -1, dtype=torch.int32, device=dev)
        self.states = torch.zeros(B, T, info.n_layers, info.d_state, dtype=torch.int8, device=dev)
        init = np.full(B, O.DIGEST_INIT, np.uint64).view(np.int64)
        self.digest = torch.as_tensor(init, device=dev)
        L = _lib.lib()
        self.fn = getattr(L, entry)
        self.model, self.B, self.T = model, B, T

    def launch(self):
        import torch
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        return self.fn(self.model._h, p(self.x), self.B, self.T, p(self.state), p(self.logits), p(self.leaves),
                       p(self.states), p(self.digest), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))

    def host(self):
        import torch
        torch.cuda.synchronize()
        return {"logits": self.logits.cpu().numpy(), "leaves": self.leaves.cpu().numpy(),
                "states": self.states.cpu().numpy(), "state": self.state.cpu().numpy(),
                "digest": self.digest.cpu().numpy()}


def _run(model, x, entry):
    from yggdrasil_amd import _lib
    c = _Call(model, x, entry)
    _lib.check(c.launch())
    return c.host()


def _same(a, b, what):
    for k in ("logits", "leaves", "states", "state", "digest"):
        if not np.array_equal(a[k], b[k]):
            bad = np.argwhere(a[k] != b[k])
            raise AssertionError(f"{what}: {k} differs at {bad[:4].tolist()} ({len(bad)} entries)")


@pytest.fixture(scope="module")
def skew_model(tmp_path_factory):
    path = tmp_path_factory.mktemp("noalloc") / "grp_8_256_4_skew.bin"
    synth.write_model(synth.ModelSpec(128, 16, 8, 256, 4, router="skew"), 5, path)
    return path


def test_noalloc_matches_grouped(skew_model):
    from yggdrasil_amd.inference import Yggdrasil
    model = Yggdrasil.load(skew_model)
    assert model.info.grouped == 1
    for B, T, seed in ((300, 6, 1), (120, 3, 2)):
        _say(f"noalloc B={B} T={T}")
        x = np.ascontiguousarray(synth.zipf_bytes(B, T, seed), np.int32)
        got = _run(model, x, "ygg_run_grouped_noalloc")
        want = _run(model, x, "ygg_run_grouped")
        _same(got, want, f"B={B} T={T}")
        ref = O.Oracle(skew_model).run(x, states=True, digest=True)
        _same(got, {**ref, "digest": ref["digest"].view(np.int64)}, f"B={B} T={T} oracle")
    assert model.take_errors() == 0
    model.close()


def test_noalloc_graph_replay(skew_model):
    """The call captured in a hipGraph on a model that has made no grouped call before, replayed twice with eager
    work and a sync between replays; every replay equals the eager grouped call."""
    import torch
    from yggdrasil_amd import _lib
    from yggdrasil_amd.inference import Yggdrasil
    model = Yggdrasil.load(skew_model)
    x = np.ascontiguousarray(synth.zipf_bytes(200, 4, 7), np.int32)
    c = _Call(model, x, "ygg_run_grouped_noalloc")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = c.launch()
    _lib.check(rc)
    want = _run(model, x, "ygg_run_grouped")
    init = torch.as_tensor(np.full(200, O.DIGEST_INIT, np.uint64).view(np.int64), device=model.device)
    for i in range(2):
        c.state.zero_()
        c.logits.fill_(-1.0)
        c.leaves.fill_(-1)
        c.states.zero_()
        c.digest.copy_(init)
        g.replay()
        _ = torch.randn(1000, device=model.device).sum()
        _same(c.host(), want, f"replay {i}")
    model.close()


@pytest.mark.timeout(300)
def test_noalloc_config5_streams_and_limit():
    """8192 streams of the configuration-5 model (16 tokens) equal ygg_run_grouped; 12 000 streams exceed the static
    workspace and are refused with YGG_ERR_LIMITS before anything runs."""
    import os
    from pathlib import Path
    import torch
    from yggdrasil_amd import _lib
    from yggdrasil_amd.inference import Yggdrasil
    w = synth.CONFIGS[5]
    cache = Path(os.environ.get("YGG_BENCH_DIR", "/tmp/ygg_bench"))
    cache.mkdir(parents=True, exist_ok=True)
    path = cache / f"{w.name}_seed{w.model_seed}.bin"
    if not path.exists():
        tmp = path.with_suffix(".tmp")
        synth.write_model(w.spec, w.model_seed, tmp)
        os.replace(tmp, path)
    model = Yggdrasil.load(path)
    x = w.make_tokens(8192, 16)
    _say("noalloc config 5: 8192 x 16")
    _same(_run(model, x, "ygg_run_grouped_noalloc"), _run(model, x, "ygg_run_grouped"), "config 5")
    big = _Call(model, np.zeros((12000, 1), np.int32), "ygg_run_grouped_noalloc")
    rc = big.launch()
    assert _lib.ERRORS[rc] == "limits", rc
    assert b"static" in _lib.lib().ygg_last_error()
    torch.cuda.synchronize()
    assert model.take_errors() == 0
    model.close()
