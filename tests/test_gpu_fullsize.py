"""Parity at the benchmark configurations' full sizes: one ygg_run launch over all B streams x T tokens of
configurations 2-5 (the launch bench.py times, with the kernel the library picks for it), checked against the C oracle
over every stream and token through two size-independent sums: the digest of every leaf and int8 state (per stream,
order-sensitive) and the sum of the f32 bit patterns of every logit (per stream). Both are exact integer checks: one
differing leaf, state byte or logit bit changes them.

Config 1 (one stream of 4096 tokens) is checked token by token in test_gpu_parity.py.
"""
import os
import time
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from yggdrasil_amd import synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _model(cfg) -> Path:
    """The model file of configuration cfg (an int), or of configuration 4 with its routed inputs stored factored at
    rank 64 ("4f": bench.py --storage factored)."""
    w = _workload(cfg)
    cache = Path(os.environ.get("YGG_BENCH_DIR", "/tmp/ygg_bench"))
    cache.mkdir(parents=True, exist_ok=True)
    p = cache / f"{w.name}_seed{w.model_seed}.bin"
    if not p.exists():
        tmp = p.with_suffix(".tmp")
        synth.write_model(w.spec, w.model_seed, tmp)
        os.replace(tmp, p)
    return p


def _gpu_sums(model, x: np.ndarray, digest: bool = True):
    """One launch over all of x; per-stream digest (None without: the plain run build, the one bench.py times), logit
    bit sums and final states."""
    import torch
    B, T = x.shape
    xt = torch.as_tensor(x, device=model.device).contiguous()
    r = model.run(xt, digest=digest)
    torch.cuda.synchronize()
    assert model.take_errors() == 0
    lg = r["logits"]
    sums = torch.empty(B, dtype=torch.int64, device=model.device)
    step = max(1, (1 << 28) // max(1, T * model.vocab))
    for b0 in range(0, B, step):
        bits = lg[b0:b0 + step].view(torch.int32).to(torch.int64) & 0xFFFFFFFF
        sums[b0:b0 + step] = bits.sum(dim=(1, 2))
    torch.cuda.synchronize()
    out = (r["digest"].cpu().numpy().view(np.uint64) if digest else None, sums.cpu().numpy().astype(np.uint64),
           r["state"].cpu().numpy())
    del r, lg
    torch.cuda.empty_cache()
    return out


def _workload(cfg):
    import dataclasses
    if cfg == "4f":
        w = synth.CONFIGS[4]
        return dataclasses.replace(w, name=w.name + "_factored", spec=dataclasses.replace(w.spec, input_rank=64))
    return synth.CONFIGS[cfg]


# The build bench.py times for each configuration's full launch (ygg_run, no digest), as bench.py's roofline.kernel
# names it; the run with a digest takes the score build of the same kernel.
TIMED = {2: "ygg::flow_kernel<64, 8, 16, 2, 3, 0, false>", 3: "ygg::flow_kernel<96, 8, 16, 3, 4, 0, false>",
         4: "ygg::fast_kernel<128, 8, 16, 4, 0, false, false, false>",
         5: "ygg::fast_kernel<128, 8, 16, 4, 0, false, true, false>"}


@pytest.mark.timeout(900)
@pytest.mark.parametrize("cfg", [2, 3, 5, 4, "4f"])
def test_full_size_digest(cfg):
    """Two launches over the full workload: the plain run build (the one bench.py times: logits and final states
    against the oracle's per-stream logit bit sums and states) and the score build (with the digest of every leaf
    and state as well)."""
    from yggdrasil_amd.inference import Yggdrasil
    w = _workload(cfg)
    path = _model(cfg)
    x = w.make_tokens()
    B, T = x.shape
    model = Yggdrasil.load(path)
    timed = model.kernel_name(B, T)
    _say(f"config {cfg}: {B} x {T}, timed kernel {timed}, digest kernel {model.kernel_name(B, T, score=True)}")
    if cfg in TIMED:
        assert timed == TIMED[cfg], timed
    t0 = time.time()
    _, ls0, st0 = _gpu_sums(model, x, digest=False)
    _say(f"config {cfg}: timed build done in {time.time() - t0:.1f}s")
    t0 = time.time()
    dg, ls, st = _gpu_sums(model, x)
    model.close()
    _say(f"config {cfg}: GPU done in {time.time() - t0:.1f}s; oracle on {min(os.cpu_count() or 1, 16)} threads")
    t0 = time.time()
    rdg, rls, rst = O.Oracle(path).run_sums(x)
    _say(f"config {cfg}: oracle done in {time.time() - t0:.1f}s")
    np.testing.assert_array_equal(st0, rst)
    bad = np.nonzero(ls0 != rls)[0]
    assert bad.size == 0, f"timed build: logit sums differ on {bad.size} of {B} streams, first {bad[:8].tolist()}"
    np.testing.assert_array_equal(st, rst)
    bad = np.nonzero(dg != rdg)[0]
    assert bad.size == 0, f"digest differs on {bad.size} of {B} streams, first {bad[:8].tolist()}"
    bad = np.nonzero(ls != rls)[0]
    assert bad.size == 0, f"logit sums differ on {bad.size} of {B} streams, first {bad[:8].tolist()}"


@pytest.mark.timeout(600)
@pytest.mark.parametrize("cfg", [3, 4])
def test_few_streams_full_model(cfg, monkeypatch):
    """The few-stream kernels on the full configuration 3 and 4 models (D = 13 and 14: the deep descent ends in one
    round of 63 nodes): 6 streams x 40 tokens through the kernel the library picks (layer-pipelined) and greedy
    generation (the deep kernel), then through the deep kernel forced for every call (one launch, launches of 3
    tokens, a step loop). Every leaf, state after every token, logit and generated token equals the oracle's."""
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    w = synth.CONFIGS[cfg]
    path = _model(cfg)
    x = w.make_tokens(6, 40)
    orc = O.Oracle(path)
    ref = orc.run(x, states=True)

    def same(got, what):
        for k in ("leaves", "states", "logits"):
            a, b = got[k], ref[k][:, :got[k].shape[1]]
            assert np.array_equal(a, b), f"config {cfg} {what}: {k} differs at {np.argwhere(a != b)[:4].tolist()}"

    monkeypatch.delenv("YGG_DEEP", raising=False)
    for k in ("auto", "deep"):
        if k == "auto":
            monkeypatch.delenv("YGG_KERNEL", raising=False)
        else:
            monkeypatch.setenv("YGG_KERNEL", k)
        model = Yggdrasil.load(path)
        assert model.info.deep == 1 and model.info.kernel == 1
        assert model.info.deep_max_streams > 0
        _say(f"config {cfg}: 6 x 40, kernel {k}, pipe_max {model.info.pipe_max_streams}, "
             f"deep_max {model.info.deep_max_streams}")
        r = model.run(x, leaves=True, states=True)
        torch.cuda.synchronize()
        same({key: v.cpu().numpy() for key, v in r.items()}, f"{k} one launch")
        if k == "auto":
            # greedy generation of 12 tokens after a 4-token prompt (the deep kernel): the oracle's argmax loop
            out = model.generate(x[:, :4], 12, temperature=0)
            r0 = orc.run(x[:, :4])
            lg, st = r0["logits"][:, -1], r0["state"]
            for i in range(12):
                tok = lg.argmax(-1).astype(np.int32)
                assert np.array_equal(out[:, 4 + i], tok), (cfg, i)
                r1 = orc.run(tok[:, None], state=st)
                lg, st = r1["logits"][:, 0], r1["state"]
        if k == "deep":
            parts, st = [], None
            for t0 in range(0, 39, 3):
                rr = model.run(x[:, t0:t0 + 3], state=st, leaves=True, states=True)
                parts.append({key: v.cpu().numpy() for key, v in rr.items()})
                st = rr["state"]
            same({key: np.concatenate([p[key] for p in parts], 1) for key in ("leaves", "states", "logits")},
                 "deep 3-token launches")
            st = model.init_state(6)
            for t in range(6):
                lg, st = model.step(x[:, t], st)
                assert np.array_equal(lg.cpu().numpy(), ref["logits"][:, t]), (cfg, t)
                assert np.array_equal(st.cpu().numpy(), ref["states"][:, t]), (cfg, t)
        model.close()
        torch.cuda.empty_cache()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("cfg", [3, 4])
def test_spec_generation_full_model(cfg, monkeypatch):
    """Greedy generation of one stream on the full configuration 3 and 4 models through the speculating build (the
    one bench.py's batch-1 leg times): 256 tokens after a 4-token prompt. Every token and every logit equals the
    oracle's argmax loop, and the helpers served the steps (nearly every step taken from a slot)."""
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    for k in ("YGG_KERNEL", "YGG_SPEC", "YGG_SPEC_EPOCH", "YGG_SPEC_HELPERS"):
        monkeypatch.delenv(k, raising=False)
    w = synth.CONFIGS[cfg]
    path = _model(cfg)
    steps = 256
    model = Yggdrasil.load(path)
    name = model.kernel_name(1, steps, generate=True)
    _say(f"config {cfg}: speculating generation, {name}")
    assert name.startswith("ygg::fast_kernel<") and name[len("ygg::fast_kernel<"):-1].split(", ")[4] == "5", name
    prompt = w.make_tokens(1, 4)[0]
    model.spec_stats(reset=True)
    out, lg = model.generate(prompt, steps, temperature=0, return_logits=True)
    torch.cuda.synchronize()
    st = model.spec_stats()
    _say(f"  stats {st}")
    orc = O.Oracle(path)
    r = orc.run(prompt[None, :])
    olg, ost = r["logits"][:, -1], r["state"]
    for i in range(steps):
        tok = olg.argmax(-1).astype(np.int32)
        assert out[4 + i] == tok[0], (cfg, i, int(out[4 + i]), int(tok[0]))
        np.testing.assert_array_equal(lg[0, i].cpu().numpy(), olg[0], err_msg=f"config {cfg} step {i}")
        if i + 1 < steps:
            r = orc.run(tok[:, None], state=ost)
            olg, ost = r["logits"][:, 0], r["state"]
    assert st["hits"] + st["misses"] == steps - 1, st
    assert st["hits"] >= steps - 8 and st["helpers_timed_out"] == 0, st
    model.close()
    torch.cuda.empty_cache()


@pytest.mark.timeout(600)
def test_reference_large_shape_full_model():
    """The reference's largest trained shape (configs/enwik8/large.yaml: 5 layers, d = 256, D = 10, R = 32, R2 = 64;
    a random 0.68 GB model of the 681 MB published file's size) over 512 streams x 256 Zipf tokens in one launch, on
    the kernel the library picks, against the C oracle's per-stream digest and logit sums."""
    from yggdrasil_amd.inference import Yggdrasil
    cache = Path(os.environ.get("YGG_BENCH_DIR", "/tmp/ygg_bench"))
    cache.mkdir(parents=True, exist_ok=True)
    path = cache / "ref_large_d256_L5_D10_seed5.bin"
    if not path.exists():
        tmp = path.with_suffix(".tmp")
        synth.write_model(synth.ModelSpec(256, 16, 10, 256, 5, 32, 64, router="gauss"), 5, tmp)
        os.replace(tmp, path)
    x = synth.zipf_bytes(512, 256, 7)
    model = Yggdrasil.load(path)
    assert model.info.kernel == 1
    _say(f"large shape: 512 x 256, kernel {model.kernel_name(512, 256)}")
    dg, ls, st = _gpu_sums(model, x)
    model.close()
    rdg, rls, rst = O.Oracle(path).run_sums(x)
    np.testing.assert_array_equal(st, rst)
    assert (dg == rdg).all() and (ls == rls).all()
