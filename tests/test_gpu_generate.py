"""GPU parity of the fused generate (ygg_generate through Yggdrasil.generate): sampling on the device, every sampled
token fed back as the next input within one launch.

Greedy generation equals the oracle's step loop with argmax (the reference's generate, yggdrasil/inference.py:190-202)
token for token, and every logit it sampled from equals the oracle's bit for bit. Sampled generation is replayed
through the oracle (its logits must equal the oracle's on the sequence it produced) and each token is checked
against the float64 restatement of the sampler (oracle.sample) with the same uniform, up to float32 rounding at a
CDF boundary; draws over many streams follow softmax(logits / temperature) within the top_k classes.
"""
import numpy as np
import pytest

from oracle import oracle as O
from yggdrasil_amd import synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(params=["fast", "deep", "generic"])
def kernel_env(request, monkeypatch):
    """Generation runs on the per-stream kernels only (the layer-pipelined one overlaps tokens): force each (deep: one
    stream per workgroup with the deep router descent, which the library picks for few streams)."""
    monkeypatch.setenv("YGG_KERNEL", request.param)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    return request.param


@pytest.fixture(scope="module")
def gmodel(model_dir):
    spec = synth.ModelSpec(128, 16, 10, 256, 4, router="gauss")
    path = model_dir / "gen_c4small.bin"
    if not path.exists():
        synth.write_model(spec, 11, path)
    return path


def _load(path, kernel_env):
    from yggdrasil_amd.inference import Yggdrasil
    m = Yggdrasil.load(path)
    assert m.info.kernel == (0 if kernel_env == "generic" else 1), m.info.kernel
    assert (m.info.deep_max_streams > 0) == (kernel_env in ("deep", "auto")), m.info.deep_max_streams
    want = {"auto": "ygg::fast_kernel<", "deep": "ygg::fast_kernel<",
            "fast": "ygg::fast_kernel<", "generic": "ygg::run_kernel<"}[kernel_env]
    assert m.kernel_name(8, 32, generate=True).startswith(want), m.kernel_name(8, 32, generate=True)
    return m


def _oracle_greedy(orc, prompt, n):
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


def test_generate_greedy_equals_oracle(gmodel, kernel_env):
    import torch
    _say(f"greedy kernel {kernel_env}")
    prompt = synth.zipf_bytes(6, 9, 21)
    n = 40
    model = _load(gmodel, kernel_env)
    out, lg = model.generate(prompt, n, temperature=0, return_logits=True)
    torch.cuda.synchronize()
    orc = O.Oracle(gmodel)
    want, want_lg = _oracle_greedy(orc, prompt, n)
    np.testing.assert_array_equal(out[:, :9], prompt)
    np.testing.assert_array_equal(out[:, 9:], want)
    np.testing.assert_array_equal(lg.cpu().numpy(), want_lg)
    # one stream, 1-d prompt; a one-token prompt starts from the zero state
    one = model.generate(prompt[2], 12, temperature=0)
    np.testing.assert_array_equal(one, out[2, :21])
    w1, _ = _oracle_greedy(orc, prompt[:, :1], 5)
    np.testing.assert_array_equal(model.generate(prompt[:, :1], 5, temperature=0)[:, 1:], w1)
    np.testing.assert_array_equal(model.generate(prompt, 0), prompt)
    model.close()


@pytest.mark.parametrize("temperature,top_k,seed", [(1.0, 0, 0), (0.7, 20, 5), (1.5, 3, 2 ** 63 + 9)])
def test_generate_sampled_replays_through_oracle(gmodel, kernel_env, temperature, top_k, seed):
    import torch
    _say(f"sampled T={temperature} k={top_k} seed={seed} kernel {kernel_env}")
    prompt = synth.zipf_bytes(8, 5, 4)
    n = 32
    model = _load(gmodel, kernel_env)
    out, lg = model.generate(prompt, n, temperature=temperature, top_k=top_k, seed=seed, return_logits=True)
    torch.cuda.synchronize()
    lg = lg.cpu().numpy()
    toks = out[:, 5:]
    # the logits each token was drawn from are the oracle's on the sequence generated so far
    ref = O.Oracle(gmodel).run(out[:, :-1].astype(np.int32))
    np.testing.assert_array_equal(lg, ref["logits"][:, 4:])
    close = 0
    for b in range(out.shape[0]):
        for t in range(n):
            c, margin = O.sample(lg[b, t], temperature, top_k, O.sample_uniform(seed, b, t))
            if margin > 1e-4:
                assert toks[b, t] == c, (b, t, toks[b, t], c, margin)
            else:
                close += 1
            if top_k:
                assert lg[b, t, toks[b, t]] >= np.sort(lg[b, t])[-top_k]
    assert close < 4, close
    # same seed, same draws; another seed, other draws
    again = model.generate(prompt, n, temperature=temperature, top_k=top_k, seed=seed)
    np.testing.assert_array_equal(again, out)
    other = model.generate(prompt, n, temperature=temperature, top_k=top_k, seed=seed + 1)
    assert not np.array_equal(other, out)
    model.close()


@pytest.mark.parametrize("which", ["medium", "large", "c4shape_5layers"])
def test_generate_without_deep_build(model_dir, monkeypatch, which):
    """Models whose deep build does not fit a workgroup's LDS (the reference's medium and large shapes at 5 layers,
    configuration 4's shape at 5 layers) generate few streams on the generate build with the one-token build's
    descent: its second round folded into the tail (three-round plans of at most 6 levels after the first: D = 10),
    else read from global memory (D = 12: rounds 4, 4, 4). Greedy tokens and the logits they come from equal the
    oracle's argmax loop; sampled tokens' logits replay through the oracle and each token is the sampler's."""
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    spec = {"medium": synth.ModelSpec(128, 16, 10, 27, 5, 16, 32, router="gauss"),
            "large": synth.ModelSpec(256, 16, 10, 27, 5, 32, 64, router="gauss"),
            "c4shape_5layers": synth.ModelSpec(128, 16, 12, 256, 5, router="gauss")}[which]
    path = model_dir / f"gen_one_{which}.bin"
    if not path.exists():
        synth.write_model(spec, 19, path)
    model = Yggdrasil.load(path)
    assert model.info.deep_max_streams == 0
    name = model.kernel_name(6, 40, generate=True)
    _say(f"generation without a deep build, {which}: {name}")
    assert name.startswith(f"ygg::fast_kernel<{spec.d_state}, ") and ", 4, false, false, " in name, name
    assert ", 4, false, false, " not in model.kernel_name(1 << 20, 40, generate=True)
    assert ", 4, false, false, " not in model.kernel_name(6, 7, generate=True)
    prompt = synth.zipf_bytes(6, 9, 21) % spec.vocab
    n = 40
    out, lg = model.generate(prompt, n, temperature=0, return_logits=True)
    torch.cuda.synchronize()
    orc = O.Oracle(path)
    want, want_lg = _oracle_greedy(orc, prompt, n)
    np.testing.assert_array_equal(out[:, 9:], want)
    np.testing.assert_array_equal(lg.cpu().numpy(), want_lg)
    temperature, top_k, seed = 0.8, 5, 3
    out, lg = model.generate(prompt, n, temperature=temperature, top_k=top_k, seed=seed, return_logits=True)
    torch.cuda.synchronize()
    lg = lg.cpu().numpy()
    np.testing.assert_array_equal(lg, orc.run(out[:, :-1].astype(np.int32))["logits"][:, 8:])
    close = 0
    for b in range(out.shape[0]):
        for t in range(n):
            c, margin = O.sample(lg[b, t], temperature, top_k, O.sample_uniform(seed, b, t))
            if margin > 1e-4:
                assert out[b, 9 + t] == c, (b, t, out[b, 9 + t], c, margin)
            else:
                close += 1
    assert close < 4, close
    model.close()


def test_generate_beyond_deep_streams(gmodel, monkeypatch):
    """More streams than the deep kernel takes (one workgroup per CU) generate on the generation build with the
    one-token build's descent, one stream per workgroup: greedy tokens and the logits they come from equal the
    oracle's argmax loop."""
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    model = Yggdrasil.load(gmodel)
    B, n = model.info.deep_max_streams + 3, 24
    name = model.kernel_name(B, n, generate=True)
    _say(f"generation of {B} streams: {name}")
    assert name == "ygg::fast_kernel<128, 8, 16, 4, 4, false, false, false>", name
    prompt = synth.zipf_bytes(B, 3, 8)
    out, lg = model.generate(prompt, n, temperature=0, return_logits=True)
    torch.cuda.synchronize()
    want, want_lg = _oracle_greedy(O.Oracle(gmodel), prompt, n)
    np.testing.assert_array_equal(out[:, 3:], want)
    np.testing.assert_array_equal(lg.cpu().numpy(), want_lg)
    model.close()


def test_generate_distribution(gmodel, monkeypatch):
    """16384 streams from one prompt, one draw each: frequencies follow softmax(logits / T) over the top_k."""
    import torch
    from scipy import stats
    _say("distribution")
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    model = _load(gmodel, "auto")
    B = 16384
    prompt = np.tile(synth.zipf_bytes(1, 6, 8), (B, 1))
    for temperature, top_k in ((0.8, 0), (1.2, 6)):
        out, lg = model.generate(prompt, 1, temperature=temperature, top_k=top_k, seed=77, return_logits=True)
        torch.cuda.synchronize()
        lg = lg[0, 0].cpu().numpy().astype(np.float64)
        p = np.exp((lg - lg.max()) / temperature)
        if top_k:
            p[lg < np.sort(lg)[-top_k]] = 0
        p /= p.sum()
        cnt = np.bincount(out[:, -1], minlength=lg.size)
        assert cnt[p == 0].sum() == 0
        big = p * B >= 5
        f_obs = np.append(cnt[big], cnt[~big].sum())
        f_exp = np.append(p[big] * B, p[~big].sum() * B)
        keep = f_exp > 0
        assert stats.chisquare(f_obs[keep], f_exp[keep]).pvalue > 1e-4, (temperature, top_k)
    model.close()


def test_generate_errors(gmodel, monkeypatch):
    import ctypes
    import torch
    from yggdrasil_amd import _lib
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    model = _load(gmodel, "auto")
    with pytest.raises(ValueError):
        model.generate([1, 2], 3, temperature=-1)
    with pytest.raises(ValueError):
        model.generate([1, 2], 3, top_k=-2)
    with pytest.raises(ValueError):
        model.generate([1, 300], 3)
    L = _lib.lib()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.ygg_generate(model._h, None, 1, 1, None, ctypes.c_float(float("nan")), 0, 0, None, None, s) == 5
    # a first token out of range: bit 0 of the error word, that stream's output untouched
    first = torch.tensor([3, 999], dtype=torch.int32, device=model.device)
    st = model.init_state(2)
    outb = torch.full((2, 4), -7, dtype=torch.int32, device=model.device)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    _lib.check(L.ygg_generate(model._h, p(first), 2, 4, p(st), ctypes.c_float(0.0), 0, 0, p(outb), None, s))
    assert model.take_errors() == 1
    o = outb.cpu().numpy()
    assert (o[1] == -7).all() and (o[0] >= 0).all()
    # 10 tokens: the speculating build (one stream), the deep build (B at most the CUs) and the generate build past
    # it (more streams): a first token out of range stops that stream only (bit 0, its outputs untouched), the
    # others generate the oracle's argmax loop
    orc = O.Oracle(gmodel)
    cus = model.info.deep_max_streams
    assert cus > 0
    for B in (1, 5, cus + 3):
        kname = model.kernel_name(B, 10, generate=True)
        _say(f"bad first token, B {B}: {kname}")
        rng = np.random.default_rng(B)
        good = rng.integers(0, 256, B).astype(np.int32)
        bad = B // 2
        first = torch.as_tensor(good, device=model.device).clone()
        first[bad] = 999
        st = model.init_state(B)
        outb = torch.full((B, 10), -7, dtype=torch.int32, device=model.device)
        _lib.check(L.ygg_generate(model._h, p(first), B, 10, p(st), ctypes.c_float(0.0), 0, 0, p(outb), None, s))
        assert model.take_errors() == 1, B
        o = outb.cpu().numpy()
        assert (o[bad] == -7).all(), B
        keep = np.array([b for b in range(B) if b != bad], dtype=np.int64)
        if keep.size:
            want, _ = _oracle_greedy(orc, good[keep][:, None], 10)
            np.testing.assert_array_equal(o[keep], want, err_msg=f"B {B}")
    model.close()
