"""GPU parity: the gfx950 step through the C-ABI against the CPU oracle, bit-exact.

Leaves, int8 states (after every token and layer) and f32 logits must equal the oracle's exactly; the oracle is
pinned to the reference kernel (cpu/ygg.cpp) in tests/test_oracle.py. Shapes: the 17 shapes of the reference's
kernel test (cpu/tests/test_kernel.py:22-33, seed 7, 8 streams x 64 tokens, zero state per stream), the benchmark
configurations at reduced stream counts, and edge cases (empty batch, zero tokens, aliased state, bad tokens,
carried state, graph replay).
"""
import ctypes
import dataclasses
import os

import numpy as np
import pytest

from oracle.oracle import Oracle
from yggdrasil_amd import synth

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def hip():
    import torch  # noqa: F401
    from yggdrasil_amd.inference import Yggdrasil
    return Yggdrasil


def _compare(got, ref, keys=("leaves", "states", "logits")):
    for k in keys:
        a, b = got[k], ref[k]
        assert a.shape == b.shape, (k, a.shape, b.shape)
        if not np.array_equal(a, b):
            bad = np.argwhere(a != b)
            raise AssertionError(f"{k}: {len(bad)} mismatches, first at {bad[:4].tolist()}: "
                                 f"gpu {a[tuple(bad[0])]} oracle {b[tuple(bad[0])]}")


@pytest.fixture(params=["flow", "pipe", "fast", "deep", "generic"])
def kernel_env(request, monkeypatch):
    """Load models with one kernel forced for every call (YGG_KERNEL): the tick-pipelined one (flow: models of 2 or
    more layers, else the per-stream one), the layer-pipelined one, the specialised per-stream one (4 streams per
    workgroup), its one-stream-per-workgroup form with the deep router descent (deep: models whose router plan allows
    it, else the per-stream one), or the general one; all but the last apply only to the specialised shapes."""
    monkeypatch.setenv("YGG_KERNEL", request.param)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    return request.param


def _gpu_run(model, x, state=None, states=True):
    import torch
    r = model.run(x, state=state, leaves=True, states=states)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in r.items()}


@pytest.mark.parametrize("ci", range(len(synth.KERNEL_CASES)))
def test_kernel_case(hip, model_dir, ci, kernel_env):
    spec = synth.KERNEL_CASES[ci]
    _say(f"case {ci}: {spec} kernel {kernel_env}")
    path = model_dir / f"kernel{ci}.bin"
    synth.write_model(spec, synth.KERNEL_SEED, path)
    x = synth.kernel_tokens(spec.vocab)
    ref = Oracle(path).run(x, states=True)
    model = hip.load(path)
    common = specialised(spec)
    if common:
        _expect_kernel(model, kernel_env)
    elif fast_only(spec):
        _expect_fast_only(model, kernel_env, spec)
    else:
        assert model.info.kernel == 0 and model.info.pipe_max_streams == 0 and model.info.deep_max_streams == 0
    got = _gpu_run(model, x)
    _compare(got, ref)
    np.testing.assert_array_equal(got["state"], ref["state"])
    model.close()


@pytest.fixture(scope="module")
def c12(model_dir):
    w = synth.CONFIGS[2]
    path = model_dir / "c12.bin"
    synth.write_model(w.spec, w.model_seed, path)
    return path


# the specialised kernels' shapes (state width, readout rank, layer-input rank; csrc/ygg_launch.h YGG_SHAPES)
SHAPES = {(64, 8, 16), (96, 8, 16), (128, 8, 16), (128, 16, 32), (256, 32, 64)}


def specialised(spec) -> bool:
    """Whether a model runs on the specialised kernels: a shape of SHAPES (a one-layer model at readout rank 8 with
    any layer-input rank), block 16, table storage or factored storage of input rank <= 64, tensor scales or group
    scales (state width 64, 128 or 256), at most 5 layers."""
    r2 = 16 if spec.n_layers == 1 else spec.layer_input_rank
    return (spec.d_state, spec.readout_rank, r2) in SHAPES and spec.block_size == 16 and spec.input_rank <= 64 and \
        (not spec.group or spec.d_state != 96) and spec.n_layers <= 5


# the per-stream kernel's other shapes (state width, readout rank, layer-input rank, block; csrc/ygg_launch.h
# YGG_FAST_EXTRA, YGG_FACT_EXTRA): the kernel-test shapes outside SHAPES or at block 8, 2 to 5 layers
FAST_ONLY = {(128, 16, 32, 8), (64, 8, 0, 8), (256, 16, 48, 8), (128, 16, 4, 16), (256, 8, 20, 16), (64, 8, 0, 16),
             (64, 32, 20, 16)}
FACT_ONLY = {(128, 16, 16, 16), (64, 8, 0, 8)}


def fast_only(spec) -> bool:
    """Whether a model runs on the per-stream kernel alone (a shape of FAST_ONLY, or of FACT_ONLY with factored
    inputs of rank <= 64; the block-8 builds at block 8)."""
    shape = (spec.d_state, spec.readout_rank, spec.layer_input_rank, spec.block_size)
    return (not specialised(spec) and 2 <= spec.n_layers <= 5 and not (spec.group and spec.d_state == 96) and
            (shape in FACT_ONLY and 0 < spec.input_rank <= 64 if spec.input_rank else shape in FAST_ONLY))


def _expect_fast_only(model, kernel_env, spec):
    """A fast-only shape: every call on the per-stream kernel (any YGG_KERNEL but generic, which forces the general
    one); no other family is built for it."""
    info = model.info
    assert info.kernel == (0 if kernel_env == "generic" else 1), info.kernel
    assert info.pipe_max_streams == info.deep_max_streams == info.flow_max_streams == 0
    assert info.grouped == 0
    family = "fact" if spec.input_rank else "fast"
    want = "ygg::run_kernel<" if kernel_env == "generic" else \
        (f"ygg::{family}8_kernel<" if spec.block_size == 8 else f"ygg::{family}_kernel<")
    for B, T in ((8, 64), (8, 1), (4096, 64)):
        assert model.kernel_name(B, T).startswith(want), model.kernel_name(B, T)
    assert model.kernel_name(8, 64, score=True).startswith(want)
    assert model.kernel_name(8, 64, generate=True).startswith(want)


def default_plan(D: int) -> list:
    """The library's default router plan: min(4, D) levels, then the rest in near-equal rounds of at most 4."""
    if D <= 0:
        return []
    h0 = min(4, D)
    rest = D - h0
    nr = (rest + 3) // 4
    return [h0] + [rest // nr + (r < rest % nr) for r in range(nr)]


def deep_plan(plan) -> bool:
    """Plans the deep descent takes: 2 to 4 rounds, the first of >= 2 levels, the third and fourth <= 6 together."""
    return 2 <= len(plan) <= 4 and plan[0] >= 2 and (len(plan) < 4 or plan[2] + plan[3] <= 6)


def flow_built(info) -> bool:
    """Models with flow_kernel builds: 2 to 5 layers, router plans of 3 or 4 rounds (depth 9 to 16)."""
    return info.n_layers > 1 and info.router_rounds in (3, 4)


def _expect_kernel(model, kernel_env):
    """The forced kernel is the one in use (the shapes passed here are all common-shape models). A model with factored
    routed inputs runs every call on fact_kernel (the specialised per-stream kernel for that storage)."""
    info = model.info
    assert info.kernel == (0 if kernel_env == "generic" else 1), info.kernel
    if info.factored and kernel_env != "generic":
        assert info.pipe_max_streams == info.deep_max_streams == info.flow_max_streams == 0
        for B, T in ((8, 64), (8, 1), (4096, 64)):
            assert model.kernel_name(B, T).startswith("ygg::fact_kernel<"), model.kernel_name(B, T)
        assert model.kernel_name(8, 64, score=True).startswith("ygg::fact_kernel<")
        assert model.kernel_name(8, 64, generate=True).startswith("ygg::fact_kernel<")
        return
    assert (info.pipe_max_streams > 0) == (kernel_env == "pipe"), info.pipe_max_streams
    plan_ok = info.n_layers > 1 and deep_plan(default_plan(info.router_depth))
    if kernel_env != "generic":
        # the deep kernel exists where its LDS fits: always for the benchmark shapes (readout rank 8, <= 4 layers)
        assert info.deep <= plan_ok, info.deep
        if plan_ok and info.readout_rank == 8 and info.n_layers <= 4:
            assert info.deep == 1
    deep = bool(info.deep)
    assert (info.deep_max_streams > 0) == (kernel_env == "deep" and deep), info.deep_max_streams
    assert (info.flow_max_streams > 0) == (kernel_env == "flow" and flow_built(info)), info.flow_max_streams
    name = model.kernel_name(8, 64)
    want = {"generic": "ygg::run_kernel<", "pipe": "ygg::pipe_kernel<", "fast": "ygg::fast_kernel<",
            "deep": "ygg::fast_kernel<", "flow": "ygg::flow_kernel<"}[kernel_env]
    if kernel_env == "flow" and not flow_built(info):
        want = "ygg::fast_kernel<"
    assert name.startswith(want), name
    if want == "ygg::flow_kernel<":
        assert name.endswith(", true>" if info.group else ", false>"), name
        return
    group = "true" if info.group else "false"
    if kernel_env in ("fast", "deep"):
        descent = "true" if kernel_env == "deep" and deep else "false"
        assert name.endswith(f", 0, {descent}, false, {group}>"), name
    if kernel_env == "pipe":
        assert name.endswith(f", 0, false, {group}>"), name
        assert model.kernel_name(8, 64, score=True).endswith(f", 2, false, {group}>")


def test_config1_full_stream(hip, c12, kernel_env):
    """Config 1: one stream of 4096 uniform bytes (the reference's CPU plumbing case), every token checked."""
    w = synth.CONFIGS[1]
    x = w.make_tokens()
    _say(f"config 1: {x.shape} kernel {kernel_env}")
    ref = Oracle(c12).run(x, states=True)
    model = hip.load(c12)
    _expect_kernel(model, kernel_env)
    _compare(_gpu_run(model, x), ref)


def test_config2_subset(hip, c12, kernel_env):
    """Config 2 at 64 streams x 512 Zipf(1.1) tokens; 66 streams for a partly filled last workgroup."""
    w = synth.CONFIGS[2]
    for B, T in ((64, 512), (66, 40)):
        x = w.make_tokens(B, T)
        _say(f"config 2: {x.shape} kernel {kernel_env}")
        ref = Oracle(c12).run(x, states=True)
        model = hip.load(c12)
        _expect_kernel(model, kernel_env)
        _compare(_gpu_run(model, x), ref)


@pytest.fixture(scope="module")
def c3(model_dir):
    w = synth.CONFIGS[3]
    path = model_dir / "c3.bin"
    synth.write_model(w.spec, w.model_seed, path)
    return path


def test_config3_subset(hip, c3, kernel_env):
    """Config 3 (V = 5, d = 96, D = 13, 3 layers) at 32 streams x 256 tokens."""
    w = synth.CONFIGS[3]
    x = w.make_tokens(32, 256)
    _say(f"config 3: {x.shape} kernel {kernel_env}")
    ref = Oracle(c3).run(x, states=True)
    model = hip.load(c3)
    _expect_kernel(model, kernel_env)
    _compare(_gpu_run(model, x), ref)


@pytest.mark.parametrize("router", ["gauss", "skew"])
def test_config4_shape_reduced(hip, model_dir, kernel_env, router):
    """The config-4/5 layer shapes (V = 256, 4 layers, d = 128, b = 16, R = 8, R2 = 16) with a depth-10 router so the
    model stays small: 64 streams x 96 Zipf tokens."""
    spec = synth.ModelSpec(128, 16, 10, 256, 4, router=router)
    path = model_dir / f"c4small_{router}.bin"
    if not path.exists():
        synth.write_model(spec, 11, path)
    x = synth.zipf_bytes(64, 96, 5)
    _say(f"config-4 shape (D=10, {router}): {x.shape} kernel {kernel_env}")
    ref = Oracle(path).run(x, states=True)
    model = hip.load(path)
    _expect_kernel(model, kernel_env)
    _compare(_gpu_run(model, x), ref)


def test_carried_state_and_step(hip, c12):
    """A launch continuing from a nonzero state; step() token by token equals one run()."""
    import torch
    w = synth.CONFIGS[2]
    x = w.make_tokens(16, 48)
    model = hip.load(c12)
    o = Oracle(c12)
    first = o.run(x[:, :16])
    ref = o.run(x[:, 16:], state=first["state"], states=True)
    st0 = torch.as_tensor(first["state"], device=model.device)
    _compare(_gpu_run(model, x[:, 16:], state=st0), ref)
    st = st0.clone()
    for t in range(16, 24):
        lg, st = model.step(x[:, t], st)
        np.testing.assert_array_equal(lg.cpu().numpy(), ref["logits"][:, t - 16])
        np.testing.assert_array_equal(st.cpu().numpy(), ref["states"][:, t - 16])


def test_step_in_place_and_edges(hip, c12):
    """ygg_step with state_in == state_out; B = 0 and T = 0 are no-ops."""
    import torch
    from yggdrasil_amd import _lib
    model = hip.load(c12)
    L = _lib.lib()
    x = synth.CONFIGS[2].make_tokens(8, 1)
    ref = Oracle(c12).run(x)
    xt = torch.as_tensor(x[:, 0], device=model.device).contiguous()
    st = model.init_state(8)
    lg = torch.empty(8, model.vocab, device=model.device)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    _lib.check(L.ygg_step(model._h, p(xt), p(st), p(st), p(lg), None, 8, s))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(lg.cpu().numpy(), ref["logits"][:, 0])
    np.testing.assert_array_equal(st.cpu().numpy(), ref["state"])
    _lib.check(L.ygg_step(model._h, None, None, None, None, None, 0, s))
    before = st.clone()
    _lib.check(L.ygg_run(model._h, p(xt), 8, 0, p(st), None, None, None, None, s))
    torch.cuda.synchronize()
    assert torch.equal(before, st)
    assert L.ygg_run(model._h, p(xt), -1, 1, p(st), None, None, None, None, s) == 5


def test_step_and_run_do_not_wait(hip, c12):
    """step() and run() return without a host synchronisation (torch's sync debug mode raises on any), with tokens
    on the GPU and with tokens on the host; a bad token already on the GPU is not read back but reported through the
    error word, while a bad host token raises before anything is launched."""
    import torch
    model = hip.load(c12)
    x = synth.CONFIGS[2].make_tokens(8, 4)
    ref = Oracle(c12).run(x, states=True)
    xd = torch.as_tensor(x, device=model.device)
    bad = xd[:, 0].clone()
    bad[3] = 999
    st = model.init_state(8)
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        lg0, st1 = model.step(xd[:, 0], st)
        lg1, st2 = model.step(x[:, 1], st1)
        r = model.run(xd[:, 2:], state=st2)
        model.step(bad, model.init_state(8))
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(lg0.cpu().numpy(), ref["logits"][:, 0])
    np.testing.assert_array_equal(lg1.cpu().numpy(), ref["logits"][:, 1])
    np.testing.assert_array_equal(r["logits"].cpu().numpy(), ref["logits"][:, 2:])
    np.testing.assert_array_equal(r["state"].cpu().numpy(), ref["state"])
    assert model.take_errors() == 1
    with pytest.raises(ValueError):
        model.step(np.array([0, 1, 2, 3, 999, 5, 6, 7]), st)
    strict = hip.load(c12, check_tokens=True)
    with pytest.raises(ValueError):
        strict.step(bad, strict.init_state(8))


def test_bad_token_stops_stream(hip, c12, kernel_env):
    """A token outside [0, V) stops its stream at that token and sets the error word; other streams go on."""
    import torch
    from yggdrasil_amd import _lib
    model = hip.load(c12)
    x = synth.CONFIGS[2].make_tokens(4, 8)
    bad = x.copy()
    bad[1, 5] = 999
    ref = Oracle(c12).run(x)
    ref_bad_prefix = Oracle(c12).run(x[1:2, :5])
    xt = torch.as_tensor(bad, device=model.device).contiguous()
    st = model.init_state(4)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(_lib.lib().ygg_run(model._h, ctypes.c_void_p(xt.data_ptr()), 4, 8, ctypes.c_void_p(st.data_ptr()),
                                  None, None, None, None, s))
    assert model.take_errors() == 1
    assert model.take_errors() == 0
    got = st.cpu().numpy()
    np.testing.assert_array_equal(got[[0, 2, 3]], ref["state"][[0, 2, 3]])
    np.testing.assert_array_equal(got[1], ref_bad_prefix["state"][0])
    with pytest.raises(ValueError):
        model.run(bad)


def test_digest_matches_oracle(hip, c12, kernel_env):
    import torch
    x = synth.CONFIGS[2].make_tokens(32, 64)
    model = hip.load(c12)
    _expect_kernel(model, kernel_env)
    r = model.run(x, logits=False, digest=True)
    torch.cuda.synchronize()
    ref = Oracle(c12).run(x, logits=False, leaves=False, digest=True)
    np.testing.assert_array_equal(r["digest"].cpu().numpy().view(np.uint64), ref["digest"])


def test_graph_replay(hip, c12):
    """graph=True: one captured step per batch size, replayed with eager work between replays, every replay
    equal to the eager step."""
    import torch
    x = synth.CONFIGS[2].make_tokens(8, 6)
    eager = hip.load(c12)
    g = hip.load(c12, graph=True)
    se, sg = eager.init_state(8), g.init_state(8)
    for t in range(6):
        le, se = eager.step(x[:, t], se)
        lgr, sg = g.step(x[:, t], sg)
        _ = torch.randn(1000, device=eager.device).sum()   # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(le, lgr) and torch.equal(se, sg), t


def test_unsplittable_transition_uses_general_kernel(hip, model_dir, monkeypatch):
    """A transition entry above 32639 has no signed-byte split (A16 = 256 hi + lo); such a model runs on the general
    kernel, still exactly."""
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    spec = synth.ModelSpec(64, 16, 5, 27, 3)
    layers = synth.random_layers(spec, 4)
    layers[1].transition[3, 0, 2, 5] = 32700
    path = model_dir / "unsplit.bin"
    from yggdrasil_amd import fmt
    fmt.write(layers, synth.output_bias(spec.vocab), path)
    model = hip.load(path)
    assert model.info.kernel == 0 and model.info.pipe_max_streams == 0
    x = synth.uniform_tokens(spec.vocab, 6, 32, 1)
    _compare(_gpu_run(model, x), Oracle(path).run(x, states=True))


def test_score_fused(hip, model_dir, kernel_env):
    """score(): the fused float64 negative log-likelihood equals the reference formula on the oracle's logits (to
    float64 rounding of a differently ordered sum) and the reference kernel's own `ygg score` bits per token."""
    from oracle import oracle as O
    spec = synth.ModelSpec(128, 16, 10, 256, 4, router="gauss")
    path = model_dir / "c4small_gauss.bin"
    if not path.exists():
        synth.write_model(spec, 11, path)
    w = synth.zipf_bytes(24, 65, 8)
    model = hip.load(path)
    _expect_kernel(model, kernel_env)
    bits = model.score(w)
    ref = O.Oracle(path).run(w[:, :-1])
    want = O.nll_bits(ref["logits"], w[:, 1:])
    np.testing.assert_allclose(bits, want, rtol=1e-12, atol=1e-9)
    if O.have_ref():
        bpc = O.ref_score(path, w[:, :-1], w[:, 1:])
        assert abs(bits.sum() / w[:, 1:].size - bpc) < 1e-6, (bits.sum() / w[:, 1:].size, bpc)
    # carried state: two halves scored from the state after the first equal the whole
    import torch
    first = model.run(w[:, :32], logits=False)
    part = model.score(w[:, 32:], state=first["state"])
    np.testing.assert_allclose(O.nll_bits(ref["logits"][:, 32:], w[:, 33:]), part, rtol=1e-12, atol=1e-9)
    torch.cuda.synchronize()


def test_score_bad_target(hip, c12):
    import torch
    from yggdrasil_amd import _lib
    model = hip.load(c12)
    x = torch.as_tensor(synth.CONFIGS[2].make_tokens(2, 5), device=model.device).contiguous()
    y = x.clone()
    y[0, 2] = 300
    st = model.init_state(2)
    nll = torch.zeros(2, dtype=torch.float64, device=model.device)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    _lib.check(_lib.lib().ygg_score(model._h, p(x), p(y), 2, 5, p(st), p(nll),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    assert model.take_errors() == 2


@pytest.mark.parametrize("which,plan", [
    ("c4small", None), ("c4small", "4,4,2"), ("c4small", "2,4,2,2"), ("c4small", "3,3,2,2"), ("c4small", "4,2,3,1"),
    ("c4small", "4,2,4"), ("c4small", "4,4,1,1"), ("c4small", "1,3,3,3"), ("c4small", "2,2,2,2,2"),
    ("c12", "2,2,3,3"), ("c12", "4,4,2")])
def test_deep_descent_plans(hip, model_dir, c12, monkeypatch, which, plan):
    """Router plans (YGG_ROUNDS) on d = 128 and d = 64 models with D = 10 under the deep descent (one launch of 40
    tokens, launches of 3 tokens with the state carried) and the layer-pipelined kernel; plans the deep descent does
    not take (a first round of 1 level, 5 rounds) run the per-stream kernel instead. Leaves, states after every token
    and logits equal the oracle's."""
    import torch
    if which == "c4small":
        path = model_dir / "c4small_gauss.bin"
        if not path.exists():
            synth.write_model(synth.ModelSpec(128, 16, 10, 256, 4, router="gauss"), 11, path)
    else:
        path = c12
    if plan:
        monkeypatch.setenv("YGG_ROUNDS", plan)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    x = synth.zipf_bytes(12, 40, 6)
    ref = Oracle(path).run(x, states=True)
    deep = deep_plan([int(h) for h in plan.split(",")] if plan else default_plan(10))
    for k in ("deep", "pipe"):
        monkeypatch.setenv("YGG_KERNEL", k)
        model = hip.load(path)
        _say(f"{which} plan {plan} kernel {k}: deep {model.info.deep}")
        assert model.info.deep == deep
        assert (model.info.deep_max_streams > 0) == (k == "deep" and deep)
        _compare(_gpu_run(model, x), ref)
        if k == "deep":
            parts, st = [], None
            for t0 in range(0, x.shape[1], 3):
                parts.append(_gpu_run(model, x[:, t0:t0 + 3], state=st))
                st = torch.as_tensor(parts[-1]["state"], device=model.device)
            got = {key: np.concatenate([p[key] for p in parts], 1) for key in ("leaves", "states", "logits")}
            _compare(got, ref)
        model.close()


@pytest.mark.parametrize("which,plan", [
    ("c4small", None), ("c4small", "4,4,2"), ("c4small", "2,4,2,2"), ("c4small", "4,2,3,1"), ("c4small", "4,4,1,1"),
    ("c4small", "1,3,3,3"), ("c12", None), ("c12", "2,2,3,3"), ("group", None), ("ref_small", None),
    ("ref_medium", None), ("ref_large", None), ("ref_medium5", None), ("ref_large5", None), ("c3", None)])
def test_one_token_build(hip, model_dir, c12, c3, monkeypatch, which, plan):
    """Calls of one token (ygg_step, and ygg_run with T = 1) whose streams are all resident take the one-token build
    (the deep descent with its second round read from global memory, or folded into the tail for three-round plans;
    one stream per workgroup) wherever the deep descent takes the plan: 12 streams stepped 6 tokens with the state
    carried, leaves, states and logits equal the oracle's. At 5 layers the build stages its LDS tables layer by layer
    (the stream waits for each routed layer's before its descent)."""
    import torch
    if which in ("c4small", "group"):
        path = model_dir / ("c4small_gauss.bin" if which == "c4small" else "c4small_group.bin")
        if not path.exists():
            synth.write_model(synth.ModelSpec(128, 16, 10, 256, 4, router="gauss", group=which == "group"), 11, path)
    elif which.startswith("ref_"):
        # (the reference's trained shapes: n, readout rank, layer-input rank)
        n, R, R2 = {"ref_small": (64, 8, 16), "ref_medium": (128, 16, 32), "ref_large": (256, 32, 64),
                    "ref_medium5": (128, 16, 32), "ref_large5": (256, 32, 64)}[which]
        L = 5 if which.endswith("5") else 3
        path = model_dir / f"one_{which}.bin"
        if not path.exists():
            synth.write_model(synth.ModelSpec(n, 16, 10, 256, L, readout_rank=R, layer_input_rank=R2, router="gauss"),
                              12, path)
    else:
        path = c12 if which == "c12" else c3
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    if plan:
        monkeypatch.setenv("YGG_ROUNDS", plan)
    model = hip.load(path)
    info = model.info
    name = model.kernel_name(12, 1)
    built = deep_plan([int(h) for h in plan.split(",")] if plan else default_plan(info.router_depth))
    _say(f"one-token build {which} plan {plan}: {name}")
    assert (", 3, false, false, " in name) == built, name
    assert ", 3, false, false, " not in model.kernel_name(12, 2)
    x = synth.zipf_bytes(12, 6, 7) % info.vocab
    ref = Oracle(path).run(x, states=True)
    parts, st = [], None
    for t in range(x.shape[1]):
        parts.append(_gpu_run(model, x[:, t:t + 1], state=st))
        st = torch.as_tensor(parts[-1]["state"], device=model.device)
    got = {key: np.concatenate([q[key] for q in parts], 1) for key in ("leaves", "states", "logits")}
    _compare(got, ref)
    st = torch.zeros_like(st)
    for t in range(x.shape[1]):
        lg, st = model.step(x[:, t], st)
        np.testing.assert_array_equal(lg.cpu().numpy(), ref["logits"][:, t])
        np.testing.assert_array_equal(st.cpu().numpy(), ref["states"][:, t])
    model.close()


def test_flow_beyond_resident(hip, model_dir, monkeypatch):
    """The default dispatch runs calls of >= 32 tokens of up to 8 streams per CU on the tick-pipelined kernel even
    where its workgroups are not all resident (4 layers: one per CU, so 8 rounds of workgroups): leaves, states and
    logits of every stream, and the scoring build's NLL and digest, equal the oracle's."""
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    from oracle import oracle as O
    path = model_dir / "c4small_gauss.bin"
    if not path.exists():
        synth.write_model(synth.ModelSpec(128, 16, 10, 256, 4, router="gauss"), 11, path)
    model = hip.load(path)
    info = model.info
    B = info.flow_max_streams
    T = 33
    name = model.kernel_name(B, T)
    _say(f"flow beyond resident: {B} streams x {T} tokens, {name}")
    assert name == "ygg::flow_kernel<128, 8, 16, 4, 3, 0, false>" and B >= 8 * info.deep_max_streams
    assert model.kernel_name(B, T, score=True) == "ygg::flow_kernel<128, 8, 16, 4, 3, 2, false>"
    x = synth.zipf_bytes(B, T + 1, 8)
    ref = Oracle(path).run(x[:, :-1], states=True, digest=True)
    _compare(_gpu_run(model, x[:, :-1]), ref)
    np.testing.assert_allclose(model.score(x, batch=B), O.nll_bits(ref["logits"], x[:, 1:]), rtol=1e-12, atol=1e-9)
    dg = model.run(x[:, :-1], logits=False, digest=True)["digest"].cpu().numpy().view(np.uint64)
    np.testing.assert_array_equal(dg, ref["digest"])
    model.close()


def test_default_dispatch(hip, model_dir, monkeypatch):
    """The kernel the library picks per call (ygg_kernel_name), and parity of the layer-pipelined kernel's capped
    build, which only calls with more streams than the uncapped build keeps resident reach (the per-stream kernel's
    capped build runs configurations 4 and 5 in test_gpu_fullsize.py)."""
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    path = model_dir / "c4small_gauss.bin"
    if not path.exists():
        synth.write_model(synth.ModelSpec(128, 16, 10, 256, 4, router="gauss"), 11, path)
    model = hip.load(path)
    info = model.info
    # mode 0: run, 1: generate, 2: score or a run with a digest; D = 10: a plan of 3 rounds
    fast = "ygg::fast_kernel<128, 8, 16, 4, {}, false, {}, false>"
    flow = "ygg::flow_kernel<128, 8, 16, 4, 3, {}, false>"
    # the tick-pipelined kernel up to 8 streams per CU (the CUs: deep_max_streams) for calls of >= 32 tokens, and
    # above that the per-stream kernel, not the layer-pipelined one
    assert info.router_rounds == 3 and info.flow_max_streams >= 8 * info.deep_max_streams > 0
    assert model.kernel_name(1, 64) == flow.format(0)
    assert model.kernel_name(1, 64, score=True) == flow.format(2)
    assert model.kernel_name(info.flow_max_streams, 32) == flow.format(0)
    assert model.kernel_name(info.flow_max_streams, 32, score=True) == flow.format(2)
    assert model.kernel_name(1, 31) == "ygg::pipe_kernel<128, 8, 16, 4, 0, false, false>"
    assert model.kernel_name(info.flow_max_streams + 1, 64) in (fast.format(0, "false"), fast.format(0, "true"))
    assert info.deep_max_streams > 0
    # one-token run calls whose streams are all resident on the one-token build (the deep descent, no staged second
    # round, one stream per workgroup): that build; more streams: the per-stream run build
    one = "ygg::fast_kernel<128, 8, 16, 4, 3, false, false, false>"
    assert model.kernel_name(1, 1) == one and model.kernel_name(info.deep_max_streams, 1) == one
    lo = _smallest_batch(model, 1, fast.format(0, "false"), 8 * info.deep_max_streams)
    assert (lo - 1) % info.deep_max_streams == 0 and model.kernel_name(lo - 1, 1) == one
    assert model.kernel_name(1, 1, score=True) == fast.format(2, "false")
    assert model.kernel_name(max(info.pipe_max_streams, info.flow_max_streams) + 1, 64) == fast.format(0, "false")
    assert model.kernel_name(info.pipe_max_streams + 1, 16) == fast.format(0, "false")
    assert model.kernel_name(16384, 64) == fast.format(0, "true")
    assert model.kernel_name(16384, 64, score=True) == fast.format(2, "true")
    # one stream of at least 8 tokens: the speculating build; two streams: the generate build with the deep descent;
    # under 8 tokens the per-stream generate build
    assert model.kernel_name(1, 100, generate=True) == "ygg::fast_kernel<128, 8, 16, 4, 5, true, false, false>"
    assert model.kernel_name(2, 100, generate=True) == "ygg::fast_kernel<128, 8, 16, 4, 1, true, false, false>"
    assert model.kernel_name(1, 7, generate=True) == fast.format(1, "false")
    assert model.kernel_name(1, 4, generate=True) == fast.format(1, "false")
    # more streams than the deep kernel takes: the generation build with the one-token build's descent while its
    # one-stream workgroups are all resident, then the per-stream generate build
    gen_one = "ygg::fast_kernel<128, 8, 16, 4, 4, false, false, false>"
    assert model.kernel_name(info.deep_max_streams + 1, 100, generate=True) == gen_one
    lo = _smallest_batch(model, 100, fast.format(1, "false"), 8 * info.deep_max_streams, generate=True)
    assert lo > info.deep_max_streams + 1 and model.kernel_name(lo - 1, 100, generate=True) == gen_one
    assert model.kernel_name(16384, 100, generate=True) == fast.format(1, "true")
    from yggdrasil_amd import _lib
    assert _lib.lib().ygg_kernel_name(model._h, 1, 1, 3, ctypes.create_string_buffer(128), 128) == 5   # bad mode
    # the capped pipe build: run calls take it only if the uncapped run build keeps fewer streams resident (without
    # the NLL's registers it may keep as many); score calls from the smallest batch the uncapped score build cannot
    assert model.kernel_name(info.pipe_max_streams, 16) in ("ygg::pipe_kernel<128, 8, 16, 4, 0, true, false>",
                                                            "ygg::pipe_kernel<128, 8, 16, 4, 0, false, false>")
    _check_capped_pipe_score(hip, monkeypatch, model, path, "ygg::pipe_kernel<128, 8, 16, 4, 2, {}, false>",
                             info.pipe_max_streams, 9)
    model.close()


def _smallest_batch(model, T, name, hi, score=False, generate=False):
    """The smallest stream count (<= hi, which runs on the kernel named) whose calls of T tokens run on it."""
    lo = 1
    assert model.kernel_name(hi, T, score=score, generate=generate) == name, \
        model.kernel_name(hi, T, score=score, generate=generate)
    while lo < hi:
        mid = (lo + hi) // 2
        if model.kernel_name(mid, T, score=score, generate=generate) == name:
            hi = mid
        else:
            lo = mid + 1
    return lo


def _check_capped_pipe_score(hip, monkeypatch, model, path, name, hi, seed):
    """Score calls of 11 tokens on the capped pipe build (name: '{}' for the cap): the fused NLL against the reference
    formula on the oracle's logits, and the digest of leaves and states. The library takes the capped score build from
    the smallest batch the uncapped one cannot keep resident when that lies within the pipe limit (hi); when the
    uncapped score build keeps as many streams resident, it takes the uncapped one up to hi, and YGG_KERNEL=pipe
    (every multi-token call on the pipe kernel) reaches the capped build from the uncapped build's limit on."""
    from oracle import oracle as O
    m = model
    if model.kernel_name(hi, 11, score=True) == name.format("true"):
        lo = _smallest_batch(model, 11, name.format("true"), hi, score=True)
        assert lo > 1 and model.kernel_name(lo - 1, 11, score=True) == name.format("false")
    else:
        assert model.kernel_name(hi, 11, score=True) == name.format("false")
        monkeypatch.setenv("YGG_KERNEL", "pipe")
        m = hip.load(path)
        monkeypatch.delenv("YGG_KERNEL")
        lo = _smallest_batch(m, 11, name.format("true"), 64 * hi, score=True)
        assert lo > hi and m.kernel_name(lo - 1, 11, score=True) == name.format("false")
    _say(f"capped pipe score build from {lo} streams (pipe_max {hi})")
    x = synth.zipf_bytes(lo, 12, seed)
    ref = Oracle(path).run(x[:, :-1], digest=True)
    np.testing.assert_allclose(m.score(x, batch=lo), O.nll_bits(ref["logits"], x[:, 1:]), rtol=1e-12, atol=1e-9)
    dg = m.run(x[:, :-1], logits=False, digest=True)["digest"].cpu().numpy().view(np.uint64)
    np.testing.assert_array_equal(dg, ref["digest"])
    if m is not model:
        m.close()


def test_group_scales_capped_builds(hip, model_dir, monkeypatch):
    """A group-scale model on the capped builds, which only calls with more streams than the uncapped builds keep
    resident reach: the per-stream kernel (4 tokens per stream) and the layer-pipelined kernel (score calls of 11
    tokens)."""
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_DEEP", raising=False)
    path = model_dir / "c4small_group.bin"
    if not path.exists():
        synth.write_model(synth.ModelSpec(128, 16, 10, 256, 4, router="gauss", group=True), 11, path)
    model = hip.load(path)
    info = model.info
    assert info.group
    fast_capped = "ygg::fast_kernel<128, 8, 16, 4, 0, false, true, true>"
    lo = _smallest_batch(model, 1, fast_capped, 16384)
    assert lo > info.pipe_max_streams and model.kernel_name(lo, 4) == fast_capped
    assert model.kernel_name(lo - 1, 1) == "ygg::fast_kernel<128, 8, 16, 4, 0, false, false, true>"
    _say(f"capped per-stream group build from {lo} streams")
    x = synth.zipf_bytes(lo, 4, 5)
    _compare(_gpu_run(model, x), Oracle(path).run(x, states=True))
    _check_capped_pipe_score(hip, monkeypatch, model, path, "ygg::pipe_kernel<128, 8, 16, 4, 2, {}, true>",
                             info.pipe_max_streams, 6)
    model.close()


@pytest.mark.parametrize("group", [False, True], ids=["tensor", "group"])
def test_large_shape_flow(hip, model_dir, monkeypatch, group):
    """The largest shape at 4 layers on flow_kernel, by the default dispatch (its descent waves compute the U'z
    products and keep V' in registers): leaves, states after every token and logits equal the oracle's."""
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_FLOW", raising=False)
    spec = synth.ModelSpec(256, 16, 10, 27, 4, 32, 64, group=group)
    path = model_dir / f"large4{'_group' if group else ''}.bin"
    if not path.exists():
        synth.write_model(spec, 17, path)
    model = hip.load(path)
    name = model.kernel_name(12, 40)
    _say(f"large shape, 4 layers, {'group' if group else 'tensor'}: {name}")
    assert name == f"ygg::flow_kernel<256, 32, 64, 4, 3, 0, {'true' if group else 'false'}>", name
    x = synth.uniform_tokens(spec.vocab, 12, 40, 4)
    _compare(_gpu_run(model, x), Oracle(path).run(x, states=True))
    model.close()


# the shapes of the reference's trained models (configs/{enwik8,hg38}/{small,medium,large}.yaml: 5 layers, block 16,
# router depth 10), here with a 27-symbol vocabulary so the models stay small
REFERENCE_SHAPES = {"small": synth.ModelSpec(64, 16, 10, 27, 5, 8, 16), "medium": synth.ModelSpec(128, 16, 10, 27, 5, 16, 32),
                    "large": synth.ModelSpec(256, 16, 10, 27, 5, 32, 64)}


def test_score_bad_target_nll_wave(hip, model_dir, monkeypatch):
    """A target outside the vocabulary in a score call on the largest shape at 5 layers (flow_kernel's score build,
    whose NLL runs on a wavefront of its own): the call reports error 2 and the other stream's NLL still equals the
    reference formula on the oracle's logits."""
    import math
    import torch
    from oracle import oracle as O
    from yggdrasil_amd import _lib
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    monkeypatch.delenv("YGG_FLOW", raising=False)
    spec = REFERENCE_SHAPES["large"]
    path = model_dir / "refshape_large.bin"
    if not path.exists():
        synth.write_model(spec, 13, path)
    model = hip.load(path)
    B, T = 2, 40
    assert model.kernel_name(B, T, score=True) == "ygg::flow_kernel<256, 32, 64, 5, 3, 2, false>"
    w = synth.uniform_tokens(spec.vocab, B, T + 1, 5)
    x = torch.as_tensor(w[:, :-1], device=model.device).contiguous()
    y = torch.as_tensor(w[:, 1:], device=model.device).contiguous()
    y[0, 7] = 300
    st = model.init_state(B)
    nll = torch.zeros(B, dtype=torch.float64, device=model.device)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    _lib.check(_lib.lib().ygg_score(model._h, p(x), p(y), B, T, p(st), p(nll),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))
    assert model.take_errors() == 2
    want = O.nll_bits(Oracle(path).run(w[1:, :-1])["logits"], w[1:, 1:])[0]
    np.testing.assert_allclose(nll[1].item() / math.log(2.0), want, rtol=1e-12)
    model.close()


@pytest.mark.parametrize("group", [False, True], ids=["tensor", "group"])
def test_medium_shape_capped_builds(hip, model_dir, monkeypatch, group):
    """The reference's medium shape on its capped per-stream builds (run and score), which only calls with more streams
    than the uncapped builds keep resident reach: leaves, states after every token and logits of a run, and the fused
    score, equal the oracle's."""
    import torch
    from oracle import oracle as O
    monkeypatch.delenv("YGG_KERNEL", raising=False)
    spec = dataclasses.replace(REFERENCE_SHAPES["medium"], group=group)
    path = model_dir / f"refshape_medium{'_group' if group else ''}.bin"
    if not path.exists():
        synth.write_model(spec, 13, path)
    model = hip.load(path)
    g = "true" if group else "false"
    capped = f"ygg::fast_kernel<128, 16, 32, 5, 0, false, true, {g}>"
    lo = _smallest_batch(model, 1, capped, 16384)
    B = lo + 3
    assert B > model.info.pipe_max_streams and model.kernel_name(B, 4) == capped
    assert model.kernel_name(B, 4, score=True) == f"ygg::fast_kernel<128, 16, 32, 5, 2, false, true, {g}>"
    _say(f"medium shape, {'group' if group else 'tensor'}: capped per-stream builds at {B} streams")
    x = synth.uniform_tokens(spec.vocab, B, 5, 7)
    ref = Oracle(path).run(x[:, :4], states=True)
    _compare(_gpu_run(model, x[:, :4]), ref)
    bits = model.score(x, batch=B)
    np.testing.assert_allclose(bits, O.nll_bits(ref["logits"], x[:, 1:]), rtol=1e-12, atol=1e-9)
    torch.cuda.synchronize()
    model.close()


@pytest.mark.parametrize("group", [False, True], ids=["tensor", "group"])
@pytest.mark.parametrize("name", list(REFERENCE_SHAPES))
def test_reference_model_shapes(hip, model_dir, kernel_env, name, group):
    """The reference's trained model shapes on every kernel, with tensor or group scales (the export's "auto" picks
    either): leaves, states after every token and logits equal the oracle's (12 streams x 40 tokens; one launch, and
    for the per-stream kernels a step loop over the first tokens); the fused score equals the reference formula on the
    oracle's logits and the digest of leaves and states the oracle's."""
    import torch
    from oracle import oracle as O
    spec = dataclasses.replace(REFERENCE_SHAPES[name], group=group)
    path = model_dir / f"refshape_{name}{'_group' if group else ''}.bin"
    if not path.exists():
        synth.write_model(spec, 13, path)
    x = synth.uniform_tokens(spec.vocab, 12, 40, 3)
    _say(f"{name} {spec}: kernel {kernel_env}")
    ref = Oracle(path).run(x, states=True)
    model = hip.load(path)
    assert specialised(spec)
    _expect_kernel(model, kernel_env)
    _compare(_gpu_run(model, x), ref)
    st = model.init_state(12)
    for t in range(3):
        lg, st = model.step(x[:, t], st)
        np.testing.assert_array_equal(lg.cpu().numpy(), ref["logits"][:, t])
        np.testing.assert_array_equal(st.cpu().numpy(), ref["states"][:, t])
    bits = model.score(x)
    np.testing.assert_allclose(bits, O.nll_bits(ref["logits"][:, :-1], x[:, 1:]), rtol=1e-12, atol=1e-9)
    dg = model.run(x, logits=False, digest=True)["digest"].cpu().numpy().view(np.uint64)
    np.testing.assert_array_equal(dg, Oracle(path).run(x, logits=False, leaves=False, digest=True)["digest"])
    torch.cuda.synchronize()
    model.close()
