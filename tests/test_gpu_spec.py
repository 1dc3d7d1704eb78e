"""GPU parity of generation for one stream with speculating helper workgroups (ygg_generate, B = 1, n >= 8: the
kModeGenSpec build of fast_kernel).

While the stream finishes step t, helper wavefronts on its XCD compute step t + 1's token layer and first routed
layers for every candidate token; the stream takes its sampled token's slot when every unit carries the step's tag
and computes the step itself otherwise. Results must equal the oracle's argmax loop (the reference's generate,
yggdrasil/inference.py:190-202) token for token and logit for logit whichever way each step went, and the counters
must show that the helpers did serve (otherwise the parity would be the fallback's only).
"""
import numpy as np
import pytest

from oracle import oracle as O
from yggdrasil_amd import synth

pytestmark = pytest.mark.gpu

def _is_spec(name: str) -> bool:
    """fast_kernel<N, R, R2, L, MODE, DEEP, CAP, GROUP> with MODE 5 (kModeGenSpec)"""
    return name.startswith("ygg::fast_kernel<") and name[len("ygg::fast_kernel<"):-1].split(", ")[4] == "5"


def _say(msg):
    print(msg, flush=True)


def _greedy(orc, prompt, n):
    """The oracle's greedy loop after a prompt (B, P): tokens (B, n) and the logits each was taken from."""
    r = orc.run(prompt)
    lg, st = r["logits"][:, -1], r["state"]
    toks, lgs = [], []
    for i in range(n):
        lgs.append(lg)
        tok = lg.argmax(-1).astype(np.int32)
        toks.append(tok)
        if i + 1 < n:
            r = orc.run(tok[:, None], state=st)
            lg, st = r["logits"][:, 0], r["state"]
    return np.stack(toks, 1), np.stack(lgs, 1)


def _model(model_dir, n, D, V, L, R=8, R2=16, group=False, router="gauss", seed=17):
    spec = synth.ModelSpec(n, 16, D, V, L, R, R2, router=router, group=group)
    path = model_dir / f"spec_{n}_{D}_{V}_{L}_{R}_{R2}_{int(group)}_{router}_{seed}.bin"
    if not path.exists():
        synth.write_model(spec, seed, path)
    return path


CASES = [
    # (d_state, depth, vocab, layers, R, R2, group): configuration 4's shape, configuration 1's, configuration 3's,
    # the reference's small shape (5 layers), other plans (8: two rounds; 10, 13: folded tails; 12: 4, 4, 4; 14: 4, 4,
    # 3, 3), group scales, a 2-layer model (one routed layer: the slot holds the token layer and layer 1's route)
    (128, 14, 256, 4, 8, 16, False),
    (64, 10, 256, 2, 8, 16, False),
    (96, 13, 5, 3, 8, 16, False),
    (64, 10, 256, 5, 8, 16, False),
    (128, 8, 27, 4, 8, 16, False),
    (128, 12, 256, 3, 8, 16, True),
    (64, 14, 256, 5, 8, 16, True),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "n{}_D{}_V{}_L{}_R{}_{}".format(*c[:5], "g" if c[6] else "t"))
def test_spec_greedy_equals_oracle(model_dir, monkeypatch, case):
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_SPEC", raising=False)
    monkeypatch.delenv("YGG_SPEC_EPOCH", raising=False)
    n, D, V, L, R, R2, group = case
    path = _model(model_dir, n, D, V, L, R, R2, group)
    model = Yggdrasil.load(path)
    assert model.info.spec_max_streams == 1, model.info.spec_max_streams
    steps = 160
    assert _is_spec(model.kernel_name(1, steps, generate=True)), model.kernel_name(1, steps, generate=True)
    assert not _is_spec(model.kernel_name(2, steps, generate=True))
    assert not _is_spec(model.kernel_name(1, 7, generate=True))
    _say(f"spec greedy {case}: {model.kernel_name(1, steps, generate=True)}")
    orc = O.Oracle(path)
    prompt = synth.zipf_bytes(1, 6, n + D)[0] if V == 256 else synth.uniform_tokens(V, 1, 6, 5)[0]
    model.spec_stats(reset=True)
    out, lg = model.generate(prompt, steps, temperature=0, return_logits=True)
    torch.cuda.synchronize()
    st = model.spec_stats()
    _say(f"  stats {st}")
    want, want_lg = _greedy(orc, prompt[None, :], steps)
    np.testing.assert_array_equal(out[6:], want[0])
    np.testing.assert_array_equal(lg.cpu().numpy()[0], want_lg[0])
    # the helpers served: most steps came from a slot; every helper with a candidate started
    assert st["hits"] + st["misses"] == steps - 1, st
    assert st["helpers_served"] > 0 and st["helpers_started"] >= min(V, 4 * 3 + 3), st
    assert st["hits"] >= (steps - 1) // 2, st
    model.close()


def test_spec_sampled_replays_and_repeats(model_dir, monkeypatch):
    """Sampled generation on the speculating build: the logits of every step equal the oracle's on the generated
    sequence, every token is the sampler's, the same seed draws the same tokens again (later calls, later epochs),
    and calls in between on other paths (several streams, a run) leave the next call's results unchanged."""
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_SPEC", raising=False)
    monkeypatch.delenv("YGG_SPEC_EPOCH", raising=False)
    path = _model(model_dir, 128, 14, 256, 4)
    model = Yggdrasil.load(path)
    prompt = synth.zipf_bytes(1, 5, 3)[0]
    steps = 96
    for temperature, top_k, seed in ((1.0, 0, 0), (0.7, 20, 5)):
        out, lg = model.generate(prompt, steps, temperature=temperature, top_k=top_k, seed=seed, return_logits=True)
        torch.cuda.synchronize()
        lg = lg.cpu().numpy()[0]
        ref = O.Oracle(path).run(out[None, :-1].astype(np.int32))
        np.testing.assert_array_equal(lg, ref["logits"][0, 4:])
        close = 0
        for t in range(steps):
            c, margin = O.sample(lg[t], temperature, top_k, O.sample_uniform(seed, 0, t))
            if margin > 1e-4:
                assert out[5 + t] == c, (t, out[5 + t], c, margin)
            else:
                close += 1
        assert close < 3, close
        model.run(synth.zipf_bytes(3, 17, 9))
        again = model.generate(prompt, steps, temperature=temperature, top_k=top_k, seed=seed)
        np.testing.assert_array_equal(again, out)
    st = model.spec_stats()
    assert st["hits"] > 0, st
    model.close()


def test_spec_epoch_wrap_and_off(model_dir, monkeypatch):
    """The epochs of a call would pass 2^32 - 1: the library clears the speculation area on the stream and starts
    again at epoch 1; the results stay the oracle's. YGG_SPEC=0 at load: no speculating build, same results."""
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_SPEC", raising=False)
    path = _model(model_dir, 128, 14, 256, 4)
    prompt = synth.zipf_bytes(1, 4, 8)[0]
    steps = 64
    want, _ = _greedy(O.Oracle(path), prompt[None, :], steps)
    monkeypatch.setenv("YGG_SPEC_EPOCH", str(2 ** 32 - 40))
    model = Yggdrasil.load(path)
    model.spec_stats(reset=True)
    for _ in range(3):          # the first call wraps, the next ones count on from 1
        out = model.generate(prompt, steps, temperature=0)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out[4:], want[0])
    assert model.spec_stats()["hits"] > 0
    model.close()
    monkeypatch.delenv("YGG_SPEC_EPOCH")
    monkeypatch.setenv("YGG_SPEC", "0")
    model = Yggdrasil.load(path)
    assert model.info.spec_max_streams == 0
    assert not _is_spec(model.kernel_name(1, steps, generate=True))
    np.testing.assert_array_equal(model.generate(prompt, steps, temperature=0)[4:], want[0])
    model.close()


@pytest.mark.parametrize("case", [(256, 0), (256, 2), (27, 4)], ids=lambda c: f"V{c[0]}_h{c[1]}")
def test_spec_fewer_helpers_than_candidates(model_dir, monkeypatch, case):
    """YGG_SPEC_HELPERS=h: h helper workgroups (2 h + 3 helper wavefronts) for more candidates than that, each helper
    taking candidate (j + step) mod V: most steps find no slot, and the stream computes them and stores their states
    into its input's slot for the next step's helpers. Greedy tokens and logits equal the oracle's, and both kinds of
    step occur."""
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_SPEC", raising=False)
    monkeypatch.delenv("YGG_SPEC_EPOCH", raising=False)
    V, h = case
    monkeypatch.setenv("YGG_SPEC_HELPERS", str(h))
    path = _model(model_dir, 128, 14 if V == 256 else 8, V, 4)
    model = Yggdrasil.load(path)
    steps = 160
    assert _is_spec(model.kernel_name(1, steps, generate=True)), model.kernel_name(1, steps, generate=True)
    orc = O.Oracle(path)
    prompt = synth.zipf_bytes(1, 6, 11)[0] if V == 256 else synth.uniform_tokens(V, 1, 6, 7)[0]
    model.spec_stats(reset=True)
    out, lg = model.generate(prompt, steps, temperature=0, return_logits=True)
    torch.cuda.synchronize()
    st = model.spec_stats()
    _say(f"spec with {h} helper workgroups, V {V}: stats {st}")
    want, want_lg = _greedy(orc, prompt[None, :], steps)
    np.testing.assert_array_equal(out[6:], want[0])
    np.testing.assert_array_equal(lg.cpu().numpy()[0], want_lg[0])
    assert st["hits"] + st["misses"] == steps - 1, st
    assert st["misses"] > 0 and st["helpers_started"] == 2 * h + 3, st
    assert st["helpers_timed_out"] == 0, st
    model.close()


@pytest.mark.parametrize("which", ["medium", "large", "c4shape_5layers"])
def test_spec_without_deep_descent(model_dir, monkeypatch, which):
    """Shapes whose deep descent does not fit LDS (the reference's medium and large shapes, configuration 4's at 5
    layers) get the speculating build with the one-token build's descent (second round folded into the tail at
    D = 8 and 10, read from global memory at D = 12), three speculated layers of five: tokens and logits equal the
    oracle's argmax loop and the helpers served."""
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_SPEC", raising=False)
    monkeypatch.delenv("YGG_SPEC_EPOCH", raising=False)
    monkeypatch.delenv("YGG_SPEC_HELPERS", raising=False)
    n, D, V, R, R2 = {"medium": (128, 10, 256, 16, 32), "large": (256, 8, 27, 32, 64),
                      "c4shape_5layers": (128, 12, 256, 8, 16)}[which]
    path = _model(model_dir, n, D, V, 5, R, R2)
    model = Yggdrasil.load(path)
    assert model.info.spec_max_streams == 1 and model.info.deep_max_streams == 0
    steps = 96
    name = model.kernel_name(1, steps, generate=True)
    assert name == f"ygg::fast_kernel<{n}, {R}, {R2}, 5, 5, false, false, false>", name
    prompt = synth.zipf_bytes(1, 4, 9)[0] if V == 256 else synth.uniform_tokens(V, 1, 4, 9)[0]
    model.spec_stats(reset=True)
    out, lg = model.generate(prompt, steps, temperature=0, return_logits=True)
    torch.cuda.synchronize()
    st = model.spec_stats()
    _say(f"spec without deep descent, {which}: {name}, stats {st}")
    want, want_lg = _greedy(O.Oracle(path), prompt[None, :], steps)
    np.testing.assert_array_equal(out[4:], want[0])
    np.testing.assert_array_equal(lg.cpu().numpy()[0], want_lg[0])
    assert st["hits"] + st["misses"] == steps - 1 and st["hits"] >= (steps - 1) // 2, st
    model.close()
