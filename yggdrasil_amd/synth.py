"""Seeded synthetic int8 models and token streams: the five benchmark configurations and the kernel-test shapes.

The distributions follow the reference's random int8 model (``cpu/export.py:487-532``): orthogonal b x b blocks times
per-row decays U[0.6, 1] as A16 = rint(2^14 A), tables U[-24, 24], router rows U[-127, 127] with thresholds
300 N(0, 1), layer-input weights U[-127, 127] (m_v = 0.05, m_ul = 0.002), readout and unembedding U[-127, 127]
(m_z = 0.002, s_q = 0.001). The draw order is this module's own, so a seed here names a different model than the
same seed in the reference; every model is a plain YGG1 file that both the reference kernel and this build read.

Two router variants serve the large benchmark models:
- ``gauss``: router rows qrow(N(0, 1/n)) (symmetric int8 per row) with small thresholds, so leaves are hit near
  uniformly (config 4);
- ``skew``: the ``gauss`` router with a forced 10-level path for ~90% of the byte values, so that most tokens land in
  16 hot leaves per routed layer (config 5).
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import numpy as np

from .fmt import SHIFT, STATE_GROUP, Factored, QuantLayer, f32, write

BIG = f32(1e30)   # a threshold no routing value crosses: forces the branch at that node


@dataclasses.dataclass(frozen=True)
class ModelSpec:
    """Shape of a random int8 model (the reference's KernelConfig, cpu/export.py:473-484, plus the router variant)."""
    d_state: int
    block_size: int
    router_depth: int
    vocab: int
    n_layers: int = 2
    readout_rank: int = 8
    layer_input_rank: int = 16
    input_rank: int = 0               # > 0: factored storage of this rank
    group: bool = False               # group scales
    router: str = "uniform"           # uniform | gauss | skew
    hot_fraction: float = 0.9         # skew: fraction of byte values forced onto the hot path
    hot_levels: int = 10              # skew: forced levels (2^(D - hot_levels) hot leaves)


def _orth_blocks(rng, b):
    q, r = np.linalg.qr(rng.standard_normal((64, b, b)))
    return q


def _router(rng, spec: ModelSpec, n: int, V: int, E: int):
    if spec.router == "uniform":
        w = rng.integers(-127, 128, (E - 1, n)).astype(np.int16)
        thr = (300 * rng.standard_normal((V, E - 1))).astype(f32)
        return w, thr
    # gauss / skew: symmetric int8 per row of N(0, 1/n) rows, small thresholds
    g = rng.standard_normal((E - 1, n)) / np.sqrt(n)
    s = np.maximum(np.abs(g).max(-1, keepdims=True), 1e-12) / 127
    w = np.rint(g / s).astype(np.int16)
    thr = (50 * rng.standard_normal((V, E - 1))).astype(f32)
    if spec.router == "skew":
        D = spec.router_depth
        levels = min(spec.hot_levels, D)
        hot = rng.permutation(V)[:int(round(spec.hot_fraction * V))]
        bits = rng.integers(0, 2, levels)
        node = 1
        for d in range(levels):
            # right iff value > thr: -BIG forces right, +BIG forces left
            thr[hot, node - 1] = -BIG if bits[d] else BIG
            node = 2 * node + int(bits[d])
    return w, thr


def random_layers(spec: ModelSpec, seed: int) -> list:
    """Random QuantLayers of shape spec (logical arrays; integers as int16/int8 to keep large models small)."""
    rng = np.random.default_rng(seed)
    n, b, D, V, R, R2 = (spec.d_state, spec.block_size, spec.router_depth, spec.vocab, spec.readout_rank,
                         spec.layer_input_rank)
    orth = _orth_blocks(rng, b)
    out = []
    for l in range(spec.n_layers):
        E = V if l == 0 else 2 ** D
        A = np.empty((E, n // b, b, b), np.int16)
        for j in range(0, E, 4096):
            m = min(4096, E - j)
            dec = rng.uniform(0.6, 1.0, (m, n // b, b, 1))
            A[j:j + m] = np.rint(2.0 ** SHIFT * dec * orth[rng.integers(0, 64, (m, n // b))])
        q = dict(token_layer=l == 0, n=n, block=b, depth=0 if l == 0 else D, transition=A)
        if l == 0:
            q["table"] = rng.integers(-24, 25, (V, 1, n), dtype=np.int16)
        else:
            if spec.input_rank:
                k = spec.input_rank
                q["factored"] = Factored(
                    input_proj=rng.integers(-127, 128, (E, n, k), dtype=np.int8),
                    input_scale=rng.uniform(0.5, 1.5, E).astype(f32),
                    bias=rng.integers(-24, 25, (E, n), dtype=np.int16),
                    token_code=rng.integers(-127, 128, (V, k), dtype=np.int8),
                    token_scale=rng.uniform(0.0002, 0.001, n).astype(f32))
            else:
                q["table"] = rng.integers(-24, 25, (E, V, n), dtype=np.int16)
            q["router_weight"], q["router_threshold"] = _router(rng, spec, n, V, E)
            q["rms_eps"] = f32(1e-4)
            if R2:
                q["layer_input_down"] = rng.integers(-127, 128, (R2, n), dtype=np.int16)
                q["layer_input_down_scale"] = np.full(R2, 0.05, f32)
                q["layer_input_proj"] = rng.integers(-127, 128, (E, n, R2), dtype=np.int8)
                q["layer_input_scale"] = f32(0.002)
        q["readout_scale"], q["unembed_scale"] = f32(0.002), f32(0.001)
        if spec.group:
            q["readout_scale"] = rng.uniform(0.0005, 0.004, (E, R)).astype(f32)
            q["unembed_scale"] = rng.uniform(0.0005, 0.002, V).astype(f32)
            if l > 0:
                q["state_r2"] = (rng.uniform(0.05, 1.0, n // STATE_GROUP) ** 2).astype(f32)
                if R2:
                    q["layer_input_scale"] = rng.uniform(0.0005, 0.004, n).astype(f32)
        q["readout"] = rng.integers(-127, 128, (E, R, n), dtype=np.int8)
        q["unembed"] = rng.integers(-127, 128, (V, R), dtype=np.int8)
        out.append(QuantLayer(**q))
    return out


def output_bias(V: int) -> np.ndarray:
    """The output bias of every synthetic model here: linspace(-1, 1, V) (as cpu/tests/test_kernel.py:39)."""
    return np.linspace(-1, 1, V)


def write_model(spec: ModelSpec, seed: int, path, bias: Optional[np.ndarray] = None) -> dict:
    """Generate and write a model; returns its header. Large record arrays are written in chunks."""
    layers = random_layers(spec, seed)
    hdr, nbytes = write(layers, output_bias(spec.vocab) if bias is None else bias, path, record_chunk=1024)
    hdr = dict(hdr, array_bytes=nbytes)
    return hdr


# ----------------------------------------------------------------------------------------------------- tokens

def uniform_tokens(V: int, B: int, T: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, V, (B, T)).astype(np.int32)


def zipf_bytes(B: int, T: int, seed: int, s: float = 1.1) -> np.ndarray:
    """Bytes with p(k) proportional to (k + 1)^-s; byte value = rank k."""
    p = (np.arange(1, 257, dtype=np.float64)) ** -s
    p /= p.sum()
    return np.random.default_rng(seed).choice(256, (B, T), p=p).astype(np.int32)


def dna_tokens(B: int, T: int, seed: int) -> np.ndarray:
    """Four symbols at 24.975% each plus a rare fifth at 0.1%."""
    p = np.array([0.24975] * 4 + [0.001])
    return np.random.default_rng(seed).choice(5, (B, T), p=p / p.sum()).astype(np.int32)


# ----------------------------------------------------------------------------------------------------- configs

@dataclasses.dataclass(frozen=True)
class Workload:
    """A benchmark configuration: model spec and seed, token generator, streams x tokens."""
    name: str
    spec: ModelSpec
    model_seed: int
    tokens: str                       # uniform | zipf | dna
    token_seed: int
    streams: int
    steps: int

    def make_tokens(self, streams: Optional[int] = None, steps: Optional[int] = None) -> np.ndarray:
        B, T = streams or self.streams, steps or self.steps
        if self.tokens == "uniform":
            return uniform_tokens(self.spec.vocab, B, T, self.token_seed)
        if self.tokens == "zipf":
            return zipf_bytes(B, T, self.token_seed)
        if self.tokens == "dna":
            return dna_tokens(B, T, self.token_seed)
        raise ValueError(self.tokens)


C12 = ModelSpec(d_state=64, block_size=16, router_depth=10, vocab=256, n_layers=2)
C3 = ModelSpec(d_state=96, block_size=16, router_depth=13, vocab=5, n_layers=3)
C4 = ModelSpec(d_state=128, block_size=16, router_depth=14, vocab=256, n_layers=4, router="gauss")
C5 = dataclasses.replace(C4, router="skew")

CONFIGS = {
    1: Workload("c1_plumbing", C12, 0, "uniform", 0, 1, 4096),
    2: Workload("c2_v256_d64", C12, 0, "zipf", 1, 1024, 2048),
    3: Workload("c3_v5_d96", C3, 2, "dna", 2, 2048, 4096),
    4: Workload("c4_v256_d128_D14", C4, 3, "zipf", 3, 4096, 1024),
    5: Workload("c5_skew", C5, 3, "uniform", 4, 8192, 512),
}

# The shapes of the reference's kernel test (cpu/tests/test_kernel.py:22-33): d_state, block_size, router_depth,
# vocab, n_layers, readout_rank, layer_input_rank (+ group scales, factored storage).
K = ModelSpec
KERNEL_CASES = [
    K(128, 16, 8, 256, 2, 8, 16), K(128, 8, 6, 256, 2, 16, 32), K(64, 16, 5, 27, 3, 32, 20),
    K(64, 8, 9, 5, 2, 8, 0), K(128, 16, 7, 5, 3, 16, 4), K(128, 16, 4, 256, 1, 8, 0),
    K(256, 16, 6, 256, 3, 32, 64), K(256, 16, 5, 5, 5, 32, 64), K(256, 8, 5, 256, 2, 16, 48),
    K(256, 16, 4, 27, 2, 8, 20),
    K(256, 16, 6, 256, 3, 32, 64, group=True), K(128, 8, 6, 256, 3, 16, 32, group=True),
    K(64, 16, 5, 5, 4, 8, 0, group=True),
    K(128, 16, 7, 256, 3, 16, 32, input_rank=32, group=True), K(256, 16, 5, 256, 3, 32, 64, input_rank=64),
    K(64, 8, 6, 5, 2, 8, 0, input_rank=16, group=True), K(128, 16, 6, 27, 2, 16, 16, input_rank=4),
]
KERNEL_SEED = 7          # cpu/tests/test_kernel.py:38
KERNEL_STREAMS, KERNEL_STEPS = 8, 64   # cpu/tests/test_kernel.py:20


def kernel_tokens(V: int) -> np.ndarray:
    """The token matrix of the reference's kernel test (cpu/tests/test_kernel.py:44-45)."""
    return np.random.default_rng(0).integers(0, V, (KERNEL_STREAMS, KERNEL_STEPS)).astype(np.int32)
