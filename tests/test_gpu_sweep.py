"""GPU parity over a seeded random sweep: models of the specialised shapes with random layer counts, router depths,
vocabularies, router kinds and tensor or group scales, run at random batch sizes (up to 2100 streams, across the
dispatch's thresholds) and token counts with each kernel forced in turn or picked by the library. Per case: leaves,
states after every token and logits of a run equal the oracle's, the fused score equals the reference formula on the
oracle's logits, and greedy generation (of up to 600 streams) equals the oracle's argmax loop. Each case prints its
parameters first. Seeds 11 and 12 draw table storage and the default router plans; seed 13 ("wide") also draws
factored routed inputs (ranks 32 and 64) and random router plans (YGG_ROUNDS, rounds of 1 to 4 levels). More seeds of
the wide draw: YGG_SWEEP_SEEDS=14,15,... (comma-separated)."""
import os
import random

import numpy as np
import pytest

from oracle import oracle as O
from oracle.oracle import Oracle
from yggdrasil_amd import synth

pytestmark = pytest.mark.gpu

# (state width, readout rank, layer-input rank): the specialised shapes
SHAPES = [(64, 8, 16), (96, 8, 16), (128, 8, 16), (128, 16, 32), (256, 32, 64)]
KERNELS = ["", "fast", "pipe", "flow", "deep", "generic"]      # "": the library's own pick


def _cases(seed: int, count: int, wide: bool = False):
    """The seed's cases; wide: factored storage and random router plans too (drawn after the others, so the cases of
    a seed without them are unchanged)."""
    rnd = random.Random(seed)
    for c in range(count):
        n, R, R2 = rnd.choice(SHAPES)
        L = rnd.randint(2, 5)
        D = rnd.randint(9, 10 if n == 256 else (12 if R == 16 else 14))
        V = rnd.choice([5, 27, 256])
        group = n != 96 and rnd.random() < 0.3
        router = rnd.choice(["uniform", "gauss", "skew"])
        u = rnd.random()
        B = rnd.randint(1, 40) if u < 0.7 else (rnd.randint(41, 600) if u < 0.9 else rnd.randint(1000, 2100))
        T = rnd.choice([1, 2, 3, 7, 31, 32, 33, 64]) if B <= 600 else rnd.choice([1, 2, 32, 33])
        kernel, mseed = rnd.choice(KERNELS), rnd.randint(0, 10 ** 6)
        K, plan = 0, ""
        if wide:
            K = rnd.choice([0, 0, 32, 64])
            if rnd.random() < 0.5:
                hs, left = [], D
                while left:
                    h = rnd.randint(1, min(4, left))
                    hs.append(h)
                    left -= h
                plan = ",".join(map(str, hs))
        yield c, synth.ModelSpec(n, 16, D, V, L, R, R2, input_rank=K, group=group, router=router), B, T, kernel, \
            mseed, plan


def _greedy_oracle(path, first: np.ndarray, n: int) -> np.ndarray:
    """n greedy tokens per row after the tokens first (B,), through the oracle a step at a time"""
    o = Oracle(path)
    st, tok, seq = None, first.astype(np.int32)[:, None], []
    for _ in range(n):
        r = o.run(tok, state=st)
        st = r["state"]
        # the first maximal class, as the device's greedy sampler
        tok = np.argmax(r["logits"][:, 0], axis=1).astype(np.int32)[:, None]
        seq.append(tok[:, 0])
    return np.stack(seq, 1)


_EXTRA = [(int(v), True) for v in os.environ.get("YGG_SWEEP_SEEDS", "").split(",") if v.strip()]


@pytest.mark.parametrize("seed,wide", [(11, False), (12, False), (13, True)] + _EXTRA)
def test_random_sweep(model_dir, monkeypatch, seed, wide):
    import torch
    from yggdrasil_amd.inference import Yggdrasil
    failures = []
    for c, spec, B, T, kernel, mseed, plan in _cases(seed, 40, wide):
        if kernel:
            monkeypatch.setenv("YGG_KERNEL", kernel)
        else:
            monkeypatch.delenv("YGG_KERNEL", raising=False)
        monkeypatch.delenv("YGG_DEEP", raising=False)
        if plan:
            monkeypatch.setenv("YGG_ROUNDS", plan)
        else:
            monkeypatch.delenv("YGG_ROUNDS", raising=False)
        tag = f"seed {seed} case {c}: {spec} B={B} T={T} kernel={kernel or 'auto'} plan={plan or 'default'}"
        print(tag, flush=True)
        path = model_dir / f"sweep{seed}_{c}.bin"
        synth.write_model(spec, mseed, path)
        x = synth.uniform_tokens(spec.vocab, B, T + 1, mseed + 1)
        ref = Oracle(path).run(x[:, :T], states=True)
        model = Yggdrasil.load(path)
        r = model.run(x[:, :T], leaves=True, states=True)
        torch.cuda.synchronize()
        for key in ("leaves", "states", "logits"):
            if not np.array_equal(r[key].cpu().numpy(), ref[key]):
                failures.append(f"{tag}: {key} on {model.kernel_name(B, T)}")
        bits = model.score(x, batch=B)
        if not np.allclose(bits, O.nll_bits(ref["logits"], x[:, 1:]), rtol=1e-12, atol=1e-9):
            failures.append(f"{tag}: score on {model.kernel_name(B, T, score=True)}")
        if T >= 2:
            G = min(B, 600)
            got = model.generate(x[:G, :1], T, temperature=0.0)[:, 1:]
            if not np.array_equal(got, _greedy_oracle(path, x[:G, 0], T)):
                failures.append(f"{tag}: generation of {G} streams on {model.kernel_name(G, T, generate=True)}")
        model.close()
        path.unlink()
    assert not failures, failures
