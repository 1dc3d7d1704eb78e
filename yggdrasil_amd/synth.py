"""Seeded synthetic int8 models and token streams: the five benchmark configurations and the kernel-test shapes.

The distributions follow the reference's random int8 model (``cpu/export.py:487-532``): orthogonal b x b blocks times
per-row decays U[0.6, 1] as A16 = rint(2^14 A), tables U[-24, 24], router rows U[-127, 127] with thresholds
300 N(0, 1), layer-input weights U[-127, 127] (m_v = 0.05, m_ul = 0.002), readout and unembedding U[-127, 127]
(m_z = 0.002, s_q = 0.001); group scales and factored storage as there. The random streams are this module's own:
every layer draws its shared arrays from one stream and its experts in fixed chunks of ``CHUNK`` experts, each chunk
from its own stream, so a 3.6 GB model is generated and packed chunk by chunk in parallel and the same seed always
gives the same file. A seed here therefore names a different model than the same seed in the reference; every model
is a plain YGG1 file that both the reference kernel and this build read.

Two router variants serve the large benchmark models:
- ``gauss``: router rows qrow(N(0, 1/n)) (symmetric int8 per row) with small thresholds 50 N(0, 1), so leaves are hit
  near uniformly (config 4);
- ``skew``: the ``gauss`` router with a forced ``hot_levels``-level path for ``hot_fraction`` of the byte values, so
  that most tokens land in 2^(D - hot_levels) hot leaves per routed layer (config 5; 16 leaves at D = 14).
"""
from __future__ import annotations

import dataclasses
import os
from concurrent.futures import ThreadPoolExecutor
from typing import Optional

import numpy as np

from .fmt import SHIFT, STATE_GROUP, Factored, QuantLayer, f32, layer_arrays, header, write_container, round_up, \
    CLASS_PAD, OUTPUT_BIAS, Streamed

BIG = f32(1e30)   # a threshold no routing value crosses: forces the branch at that node
CHUNK = 1024      # experts per random stream
_small_limit = 1 << 24   # write_model builds a layer in memory when E n (V) is at most this, else streams it


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
    hot_levels: int = 10              # skew: forced levels


def _rng(seed: int, *key) -> np.random.Generator:
    return np.random.default_rng([seed, *key])


def _orth_blocks(seed: int, b: int) -> np.ndarray:
    return np.linalg.qr(_rng(seed, 0xB10C).standard_normal((64, b, b)))[0]


def _router(rng, spec: ModelSpec, n: int, V: int, E: int):
    if spec.router == "uniform":
        w = rng.integers(-127, 128, (E - 1, n)).astype(np.int16)
        thr = (300 * rng.standard_normal((V, E - 1))).astype(f32)
        return w, thr
    g = rng.standard_normal((E - 1, n)) / np.sqrt(n)
    s = np.maximum(np.abs(g).max(-1, keepdims=True), 1e-12) / 127
    w = np.rint(g / s).astype(np.int16)
    thr = (50 * rng.standard_normal((V, E - 1))).astype(f32)
    if spec.router == "skew":
        levels = min(spec.hot_levels, spec.router_depth)
        hot = rng.permutation(V)[:int(round(spec.hot_fraction * V))]
        bits = rng.integers(0, 2, levels)
        node = 1
        for d in range(levels):
            thr[hot, node - 1] = -BIG if bits[d] else BIG   # right iff value > thr
            node = 2 * node + int(bits[d])
    return w, thr


def _experts(spec: ModelSpec, seed: int, l: int, j0: int, j1: int, orth: np.ndarray) -> dict:
    """Per-expert arrays of experts [j0, j1) of layer l (j0 a multiple of CHUNK)."""
    n, b, V, R, R2 = spec.d_state, spec.block_size, spec.vocab, spec.readout_rank, spec.layer_input_rank
    out = {k: [] for k in ("transition", "table", "readout", "layer_input_proj", "readout_scale", "input_proj",
                           "input_scale", "bias")}
    for c0 in range(j0, j1, CHUNK):
        m = min(CHUNK, j1 - c0)
        rng = _rng(seed, l, 1 + c0 // CHUNK)
        dec = rng.uniform(0.6, 1.0, (m, n // b, b, 1))
        out["transition"].append(np.rint(2.0 ** SHIFT * dec * orth[rng.integers(0, 64, (m, n // b))])
                                 .astype(np.int16))
        if l == 0:
            out["table"].append(rng.integers(-24, 25, (m, 1, n), dtype=np.int16))
        elif spec.input_rank:
            k = spec.input_rank
            out["input_proj"].append(rng.integers(-127, 128, (m, n, k), dtype=np.int8))
            out["input_scale"].append(rng.uniform(0.5, 1.5, m).astype(f32))
            out["bias"].append(rng.integers(-24, 25, (m, n), dtype=np.int16))
        else:
            out["table"].append(rng.integers(-24, 25, (m, V, n), dtype=np.int16))
        if l > 0 and R2:
            out["layer_input_proj"].append(rng.integers(-127, 128, (m, n, R2), dtype=np.int8))
        out["readout"].append(rng.integers(-127, 128, (m, R, n), dtype=np.int8))
        if spec.group:
            out["readout_scale"].append(rng.uniform(0.0005, 0.004, (m, R)).astype(f32))
    return {k: np.concatenate(v) for k, v in out.items() if v}


def _layer(spec: ModelSpec, seed: int, l: int, orth: np.ndarray, experts: Optional[dict]) -> QuantLayer:
    """QuantLayer l; the per-expert arrays come from experts (or are left as None for streamed writing)."""
    n, V, R, R2, D = spec.d_state, spec.vocab, spec.readout_rank, spec.layer_input_rank, spec.router_depth
    E = V if l == 0 else 2 ** D
    rng = _rng(seed, l, 0)
    ex = experts or {}
    q = dict(token_layer=l == 0, n=n, block=spec.block_size, depth=0 if l == 0 else D,
             transition=ex.get("transition"), readout=ex.get("readout"), table=ex.get("table"))
    if l > 0:
        if spec.input_rank:
            k = spec.input_rank
            q["factored"] = Factored(input_proj=ex.get("input_proj"), input_scale=ex.get("input_scale"),
                                     bias=ex.get("bias"), token_code=rng.integers(-127, 128, (V, k), dtype=np.int8),
                                     token_scale=rng.uniform(0.0002, 0.001, n).astype(f32))
        q["router_weight"], q["router_threshold"] = _router(rng, spec, n, V, E)
        q["rms_eps"] = f32(1e-4)
        if R2:
            q["layer_input_down"] = rng.integers(-127, 128, (R2, n), dtype=np.int16)
            q["layer_input_down_scale"] = np.full(R2, 0.05, f32)
            q["layer_input_proj"] = ex.get("layer_input_proj")
            q["layer_input_scale"] = f32(0.002)
    q["readout_scale"], q["unembed_scale"] = f32(0.002), f32(0.001)
    if spec.group:
        q["readout_scale"] = ex.get("readout_scale")
        q["unembed_scale"] = rng.uniform(0.0005, 0.002, V).astype(f32)
        if l > 0:
            q["state_r2"] = (rng.uniform(0.05, 1.0, n // STATE_GROUP) ** 2).astype(f32)
            if R2:
                q["layer_input_scale"] = rng.uniform(0.0005, 0.004, n).astype(f32)
    q["unembed"] = rng.integers(-127, 128, (V, R), dtype=np.int8)
    return QuantLayer(**q)


def random_layers(spec: ModelSpec, seed: int) -> list:
    """Random QuantLayers of shape spec, all arrays in memory (integers as int8/int16)."""
    orth = _orth_blocks(seed, spec.block_size)
    out = []
    for l in range(spec.n_layers):
        E = spec.vocab if l == 0 else 2 ** spec.router_depth
        out.append(_layer(spec, seed, l, orth, _experts(spec, seed, l, 0, E, orth)))
    return out


def output_bias(V: int) -> np.ndarray:
    """The output bias of every synthetic model here: linspace(-1, 1, V) (as cpu/tests/test_kernel.py:39)."""
    return np.linspace(-1, 1, V)


def write_model(spec: ModelSpec, seed: int, path, bias: Optional[np.ndarray] = None, threads: int = 0) -> dict:
    """Generate and write the model of (spec, seed) to path; returns its header plus array_bytes. The expert
    records are generated and packed in parallel, CHUNK experts at a time, and written in order."""
    V = spec.vocab
    orth = _orth_blocks(seed, spec.block_size)
    E_routed = 2 ** spec.router_depth
    layers = []
    for l in range(spec.n_layers):
        E = V if l == 0 else E_routed
        small = E * spec.d_state * (V if l else 1) <= _small_limit
        layers.append(_layer(spec, seed, l, orth, _experts(spec, seed, l, 0, E, orth) if small else None))
    # the header needs the shapes only: describe the streamed layers by one chunk
    probe = []
    for l, q in enumerate(layers):
        if q.transition is None:
            one = _experts(spec, seed, l, 0, 1, orth)
            probe.append(_with_experts(q, one))
        else:
            probe.append(q)
    hdr = header(probe, V)
    ob = np.zeros(round_up(V, CLASS_PAD), f32)
    ob[:V] = output_bias(V) if bias is None else bias
    arrs = [(OUTPUT_BIAS, ob)]
    nt = threads or min(16, os.cpu_count() or 1)
    for l, q in enumerate(layers):
        if q.transition is not None:
            arrs += layer_arrays(l, q, hdr)
            continue
        E = V if l == 0 else E_routed
        pl = probe[l]
        if spec.group:
            # the per-expert readout row scales are an array of their own (mzl): one pass over the chunks for them
            def scales(j0, l=l, E=E):
                return _experts(spec, seed, l, j0, min(E, j0 + CHUNK), orth)["readout_scale"]
            with ThreadPoolExecutor(nt) as ex:
                pl = dataclasses.replace(pl, readout_scale=np.concatenate(list(ex.map(scales, range(0, E, CHUNK)))))
        la = layer_arrays(l, pl, hdr)
        rec_bytes = int(dict(la)[f"l{l}_meta"][0])

        def chunks(l=l, q=q, E=E):
            def make(j0):
                j1 = min(E, j0 + CHUNK)
                part = _with_experts(q, _experts(spec, seed, l, j0, j1, orth))
                return dict(layer_arrays(l, part, hdr))[f"l{l}_rec"]
            with ThreadPoolExecutor(nt) as ex:
                yield from ex.map(make, range(0, E, CHUNK))
        arrs += [(name, Streamed(E * rec_bytes, chunks) if name == f"l{l}_rec" else a) for name, a in la]
    nbytes = write_container(path, hdr, arrs)
    return dict(hdr, array_bytes=nbytes)


def _with_experts(q: QuantLayer, ex: dict) -> QuantLayer:
    """q with its per-expert arrays replaced by ex (a chunk of experts)."""
    kw = dict(transition=ex["transition"], readout=ex["readout"], table=ex.get("table"))
    if q.factored is not None:
        kw["factored"] = dataclasses.replace(q.factored, input_proj=ex["input_proj"], input_scale=ex["input_scale"],
                                             bias=ex["bias"])
    if q.layer_input_down is not None:
        kw["layer_input_proj"] = ex["layer_input_proj"]
    if np.ndim(q.readout_scale) or "readout_scale" in ex:
        kw["readout_scale"] = ex.get("readout_scale", q.readout_scale)
    return dataclasses.replace(q, **kw)


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
