"""GPU: the float step (csrc/ygg_float.hip through ygg_float_run) against the float64 restatement oracle/float_oracle.py,
and the int8 export (yggdrasil_amd.export) whose calibration runs on the f64 kernel and whose margin search runs the
int8 kernel.

- f64 kernel: every leaf equal, logits, states and calibration maxima within 1e-10 relative of the restatement;
- f32 kernel: the reference's protocol for its float32 GPU step (cpu/tests/test_triton.py:28-67): every step from the
  restatement's state, log-probabilities within 1e-4, at most 1e-3 of the stream steps beyond (routing ties); and
  over whole sequences, logits within 2e-4 of the restatement before a stream's first route that differs from it;
- the Python API over it (Yggdrasil.load of a .npz, step, score, greedy generate) against the same restatement;
- export: the calibration maxima equal the restatement's, the written file equals quantize() on the restatement's
  maxima at the chosen margin and scale mode, and the int8 model's bits per token stay close to the float model's.
"""
import numpy as np
import pytest

from oracle import float_oracle as FO
from yggdrasil_amd import float_model as FM

pytestmark = pytest.mark.gpu

SPEC = FM.FloatSpec(d_state=64, block_size=16, router_depth=5, vocab=64, n_layers=3, router_token_dim=16,
                    input_rank=16, readout_rank=8, layer_input_rank=16)


def _say(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    p = tmp_path_factory.mktemp("float") / "m.npz"
    FM.random_checkpoint(SPEC, 21, p)
    raw, ob = FM.read(p)
    return p, FM.float_layers(raw), ob


def _tokens(B, T, seed):
    return np.random.default_rng(seed).integers(0, SPEC.vocab, (B, T))


def test_float64_kernel_equals_restatement(ckpt):
    import torch
    p, layers, ob = ckpt
    x = _tokens(16, 40, 1)
    ref = FO.run(layers, ob, x)
    m = FM.FloatYggdrasil(layers, ob, precision=64)
    r = m.run(x, leaves=True, stats=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(r["leaves"].cpu().numpy(), ref["leaves"])
    np.testing.assert_allclose(r["logits"].cpu().numpy(), ref["logits"], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(r["state"].cpu().numpy(), ref["state"], rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(r["stats"].cpu().numpy(), ref["stats"], rtol=1e-10, atol=0)
    m.close()


def test_float32_kernel_close_to_restatement(ckpt):
    import torch
    p, layers, ob = ckpt
    x = _tokens(64, 48, 2)
    ref = FO.run(layers, ob, x)
    m = FM.FloatYggdrasil(layers, ob, precision=32)
    r = m.run(x, leaves=True)
    torch.cuda.synchronize()
    lv, lg = r["leaves"].cpu().numpy(), r["logits"].cpu().numpy().astype(np.float64)
    differs = (lv != ref["leaves"]).any(-1)            # (B, T): some layer took another leaf
    split = 0
    for s in range(x.shape[0]):
        t1 = int(np.argmax(differs[s])) if differs[s].any() else x.shape[1]
        split += t1 < x.shape[1]
        np.testing.assert_allclose(lg[s, :t1], ref["logits"][s, :t1], rtol=2e-4, atol=2e-4)
    _say(f"f32: {split} of {x.shape[0]} streams leave the f64 route somewhere in {x.shape[1]} tokens")
    assert split <= 2
    m.close()


@pytest.mark.parametrize("shape", [(128, 16, 32), (256, 32, 64)], ids=["medium", "large"])
def test_float32_trained_shape_builds(shape):
    """The f32 builds specialised on the reference's medium and large trained shapes (5 layers, block 16, router depth
    10: rounds of 4, 4 and 2 levels, the first from LDS; configs/enwik8/{medium,large}.yaml), against the float64
    restatement as in test_float32_kernel_close_to_restatement. A vocabulary of 32 keeps the precomputed tables small
    (the build is picked by the shape alone)."""
    import torch
    n, R, R2 = shape
    spec = FM.FloatSpec(d_state=n, block_size=16, router_depth=10, vocab=32, n_layers=5, router_token_dim=16,
                        input_rank=64 if n == 256 else 32, readout_rank=R, layer_input_rank=R2)
    raw, ob = FM.from_params(FM.random_params(spec, 7))
    layers = FM.float_layers(raw, blas=True)
    x = np.random.default_rng(3).integers(0, spec.vocab, (8, 24))
    ref = FO.run(layers, ob, x)
    m = FM.FloatYggdrasil(layers, ob, precision=32)
    assert m.kernel_name == "ygg::float_kernel<float, %d, %d, %d, 16>" % shape, m.kernel_name
    _say(f"trained shape {shape}: {m.kernel_name}")
    r = m.run(x, leaves=True)
    torch.cuda.synchronize()
    lv, lg = r["leaves"].cpu().numpy(), r["logits"].cpu().numpy().astype(np.float64)
    differs = (lv != ref["leaves"]).any(-1)
    split = 0
    for s in range(x.shape[0]):
        t1 = int(np.argmax(differs[s])) if differs[s].any() else x.shape[1]
        split += t1 < x.shape[1]
        np.testing.assert_allclose(lg[s, :t1], ref["logits"][s, :t1], rtol=2e-4, atol=2e-4)
    _say(f"  {split} of {x.shape[0]} streams leave the f64 route somewhere in {x.shape[1]} tokens")
    assert split <= 2
    m.close()


def test_float32_step_reference_protocol(ckpt):
    """The reference's check of its float32 GPU step (cpu/tests/test_triton.py:28-67): 64 streams x 256 steps, every
    step started from the float64 state of the restatement, log-probabilities within ATOL = 1e-4, and at most
    FLIPS = 1e-3 of the stream steps beyond it (a router score within float32 rounding of 0 may turn the other way);
    score() within 1e-4 relative of the restatement's bits."""
    import torch
    B, S, ATOL, FLIPS = 64, 256, 1e-4, 1e-3
    p, layers, ob = ckpt
    x = _tokens(B, S, 6)
    m = FM.FloatYggdrasil(layers, ob, precision=32)
    ref_state = np.zeros((B, SPEC.n_layers, SPEC.d_state))
    off, worst = 0, 0.0
    for t in range(S):
        h = torch.tensor(ref_state, dtype=torch.float32, device=m.device)
        lg, _ = m.step(x[:, t], h)
        ref = FO.run(layers, ob, x[:, t:t + 1], state=ref_state)
        ref_state = ref["state"]
        l0 = ref["logits"][:, 0]
        lp0 = l0 - (np.log(np.exp(l0 - l0.max(-1, keepdims=True)).sum(-1, keepdims=True)) + l0.max(-1, keepdims=True))
        lp = torch.log_softmax(lg.double(), -1).cpu().numpy()
        d = np.abs(lp - lp0).max(-1)
        off += int((d > ATOL).sum())
        worst = max(worst, float(d[d <= ATOL].max(initial=0.0)))
    _say(f"f32 step: {off} of {B * S} stream steps beyond {ATOL}, largest difference of the others {worst:.1e}")
    assert off <= FLIPS * B * S
    w = x[:8, :129]
    ref_logits = FO.run(layers, ob, w[:, :-1])["logits"]
    mx = ref_logits.max(-1, keepdims=True)
    lse = np.log(np.exp(ref_logits - mx).sum(-1)) + mx[..., 0]
    want = (lse - np.take_along_axis(ref_logits, w[:, 1:, None], -1)[..., 0]).sum(-1) / np.log(2)
    np.testing.assert_allclose(m.score(w), want, rtol=1e-4)
    m.close()


def test_float_api(ckpt):
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    p, layers, ob = ckpt
    m = Yggdrasil.load(p, precision=64)
    assert isinstance(m, FM.FloatYggdrasil) and m.classes == SPEC.vocab
    x = _tokens(8, 20, 3)
    ref = FO.run(layers, ob, x)
    # step by step with the state carried equals the restatement
    st = m.init_state(8)
    for t in range(4):
        lg, st = m.step(x[:, t], st)
        np.testing.assert_allclose(lg.cpu().numpy(), ref["logits"][:, t], rtol=1e-10, atol=1e-10)
    # score: bits of x[:, 1:] given x[:, :-1] (yggdrasil/inference.py:179-188)
    bits = m.score(x)
    lgr = ref["logits"][:, :-1]
    mx = lgr.max(-1, keepdims=True)
    lse = np.log(np.exp(lgr - mx).sum(-1)) + mx[..., 0]
    want = (lse - np.take_along_axis(lgr, x[:, 1:, None], -1)[..., 0]).sum(-1) / np.log(2)
    np.testing.assert_allclose(bits, want, rtol=1e-9)
    # greedy generation = argmax loop of the restatement
    g = m.generate(x[:, :5], 6, temperature=0)
    seq = x[:, :5].copy()
    for _ in range(6):
        nxt = FO.run(layers, ob, seq)["logits"][:, -1].argmax(-1)
        seq = np.concatenate([seq, nxt[:, None]], 1)
    np.testing.assert_array_equal(g, seq)
    with pytest.raises(ValueError):
        m.step(np.array([SPEC.vocab] * 8), st)
    m.close()
    torch.cuda.synchronize()


def test_export_end_to_end(ckpt, tmp_path):
    import torch
    from yggdrasil_amd import export as X
    from yggdrasil_amd import fmt
    from yggdrasil_amd.inference import Yggdrasil
    p, layers, ob = ckpt
    calib = _tokens(48, 64, 4)
    out = tmp_path / "model.bin"
    rec = X.export(p, out, calib)
    _say(f"export: {rec['state_scale']} margin {rec['quantize']['hmargin']}, calibration bits {rec['calib_bpc']}")
    # the calibration maxima are the restatement's, over the input columns (the last column is only a target)
    ref_stats = FO.run(layers, ob, calib[:, :-1])["stats"]
    got = np.array([[s["state_max"], s["layer_input_max"], s["readout_max"], *s["state_group_max"],
                     *s["readout_row_max"]] for s in rec["stats"]])
    np.testing.assert_allclose(got, ref_stats, rtol=1e-10, atol=0)
    # the file is quantize() of the restatement's maxima at the chosen setting
    want = tmp_path / "want.bin"
    fmt.write(X.quantize(layers, X.stats_from_array(ref_stats, SPEC.d_state), **rec["quantize"]), ob, want,
              router_token_dim=SPEC.router_token_dim, input_rank=SPEC.input_rank)
    assert out.read_bytes() == want.read_bytes()
    # the int8 model tracks the float model on held-out windows. A random router is sensitive: once the int8 state
    # sends a stream down another leaf, its later logits are another model's, so the logits are compared on each
    # stream's tokens before its first differing leaf, where only the quantisation of the update and readout acts.
    test = _tokens(32, 64, 5)
    m8 = Yggdrasil.load(out)
    b8 = m8.score(test).sum() / test[:, 1:].size
    r8 = m8.run(test, leaves=True)
    l8, v8 = r8["logits"].double().cpu().numpy(), r8["leaves"].cpu().numpy()
    m8.close()
    mf = Yggdrasil.load(p, precision=32)
    bf = mf.score(test).sum() / test[:, 1:].size
    rf = mf.run(test, leaves=True)
    lf, vf = rf["logits"].double().cpu().numpy(), rf["leaves"].cpu().numpy()
    mf.close()
    torch.cuda.synchronize()
    differs = (v8 != vf).any(-1)
    first = np.where(differs.any(1), differs.argmax(1), test.shape[1])
    mask = np.arange(test.shape[1])[None, :] < first[:, None]
    a, b = l8[mask].ravel(), lf[mask].ravel()
    corr = np.corrcoef(a, b)[0, 1]
    rel = np.abs(a - b).mean() / lf.std()
    _say(f"held-out: bits per token float {bf:.4f} int8 {b8:.4f}; leaves equal at {(~differs).mean():.3f} of tokens, "
         f"{mask.mean():.3f} before a stream's first differing leaf; there logit correlation {corr:.5f}, mean "
         f"|dlogit| / std {rel:.4f}")
    assert abs(b8 - bf) < 0.1 * max(1.0, bf)
    assert mask.mean() > 0.05 and corr > 0.99 and rel < 0.05
