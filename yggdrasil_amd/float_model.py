"""The float inference model of a Yggdrasil checkpoint (.npz) on the GPU: the float step of yggdrasil/inference.py on
the hand-written HIP kernel of csrc/ygg_float.hip, in f32 (serving, the role of TritonYggdrasil in
yggdrasil/inference_triton.py) or f64 (the precision cpu/export.py calibrates in).

    model = FloatYggdrasil.load("run.npz")           # or Yggdrasil.load("run.npz", backend="hip")
    state = model.init_state(B)                       # (B, layers, n) float on the GPU
    logits, state = model.step(tokens, state)         # tokens (B,) -> logits (B, classes)

Checkpoint reading follows yggdrasil/inference.py:110-140 (flat "a/b/c" keys nested, old key names upgraded as
yggdrasil/config.py:84-111 lists them, unsupported layer arrays rejected); the per-layer precomputation follows
yggdrasil/inference.py:145-155 (T_r[x] = U_r v(x) + c_r; A_r = diag(clip(decay_r, -1, 1)) blockdiag(expm((G - G^T)/2)),
yggdrasil/experts.py:8-11), in float64 on the host.
"""
from __future__ import annotations

import ctypes
import dataclasses
import math
from pathlib import Path
from typing import Optional

import numpy as np

from . import _lib
from ._lib import YggError, check

LN2 = math.log(2.0)
RMS_EPS = 1e-6   # yggdrasil/config.py:8

# checkpoint keys of one layer this reader understands (yggdrasil/inference.py:33-35)
LAYER_KEYS = {"token_embed", "input_proj", "bias", "rotation", "decay", "readout", "unembed",
              "router_embed", "router_weight", "router_bias", "layer_input_down", "layer_input_proj"}
# old checkpoint key names -> current ones (the released checkpoints' names, yggdrasil/config.py:84-91)
KEY_ALIASES = {
    "root": "token_layer", "branches": "routed_layers", "head_b": "output_bias", "levels": "hre_levels",
    "v_tok": "token_embed", "u_in": "input_proj", "c": "bias", "p_out": "readout", "q_out": "unembed",
    "skew": "rotation", "d_raw": "decay", "tok": "router_embed", "w_node": "router_weight", "b_node": "router_bias",
    "v_low": "layer_input_down", "u_low": "layer_input_proj",
}


def _nest(flat: dict) -> dict:
    """{"a/b/c": array} -> nested dicts, a dict whose keys are all indices -> a list."""
    out: dict = {}
    for name, v in flat.items():
        *path, key = "/".join(KEY_ALIASES.get(p, p) for p in name.split("/")).split("/")
        d = out
        for k in path:
            d = d.setdefault(k, {})
        d[key] = np.asarray(v, np.float64)

    def lists(d):
        if not isinstance(d, dict):
            return d
        if d and all(k.isdigit() for k in d):
            return [lists(d[str(i)]) for i in range(len(d))]
        return {k: lists(v) for k, v in d.items()}
    return lists(out)


def read(path):
    """Checkpoint -> ([token layer, routed layers...] as dicts of float64 arrays, output bias (classes,))."""
    with np.load(path, allow_pickle=False) as z:
        return from_params({k: z[k] for k in z.files}, str(path))


def from_params(flat: dict, path: str = "parameters"):
    """Flat "a/b/c" parameter arrays (a checkpoint's contents) -> what read returns."""
    params = _nest(flat)
    for k in ("token_layer", "output_bias"):
        if k not in params:
            raise ValueError(f"{path}: not a Yggdrasil checkpoint (no {k})")
    layers = [params["token_layer"], *params.get("routed_layers", [])]
    for p in layers:
        if bad := set(p) - LAYER_KEYS:
            raise NotImplementedError(f"{path}: unsupported layer arrays {sorted(bad)}")
        if len(p["readout"]) != len(p["bias"]):
            raise NotImplementedError(f"{path}: the readout needs one matrix per expert")
    return layers, params["output_bias"]


def transitions(rotation: np.ndarray, decay: np.ndarray) -> np.ndarray:
    """A_r = diag(clip(decay_r, -1, 1)) blockdiag(expm((G_r - G_r^T) / 2)) -> (E, n/b, b, b), float64."""
    from scipy.linalg import expm
    gen = 0.5 * (rotation - np.swapaxes(rotation, -1, -2))
    E, g, b, _ = gen.shape
    rot = expm(gen.reshape(E * g, b, b)).reshape(E, g, b, b)
    return np.clip(decay, -1.0, 1.0).reshape(E, g, b)[..., None] * rot


@dataclasses.dataclass
class FloatLayer:
    """One layer of the float64 inference model (the arrays cpu/export.py:63-95 calls a FloatLayer)."""
    token_layer: bool
    table: np.ndarray                 # (E, V, n); token layer: (V, n), row x = T_x[x]
    transition: Optional[np.ndarray]  # (E, n/b, b, b)
    readout: np.ndarray               # (E, R, n)
    unembed: np.ndarray               # (classes, R)
    input_proj: np.ndarray            # (E, n, input_rank)
    token_embed: np.ndarray           # (V, input_rank)
    bias: np.ndarray                  # (E, n)
    router_embed: Optional[np.ndarray] = None   # (V, F)
    router_weight: Optional[np.ndarray] = None  # (2^D - 1, F [+ n])
    router_bias: Optional[np.ndarray] = None    # (2^D - 1,)
    layer_input_down: Optional[np.ndarray] = None  # (R2, n)
    layer_input_proj: Optional[np.ndarray] = None  # (E, n, R2)

    @property
    def n(self):
        return self.bias.shape[1]

    @property
    def depth(self):
        return 0 if self.token_layer else (self.router_weight.shape[0] + 1).bit_length() - 1

    @property
    def router_token_dim(self):
        return 0 if self.token_layer else self.router_embed.shape[1]

    @property
    def routes_on_state(self):
        return not self.token_layer and self.router_weight.shape[1] > self.router_embed.shape[1]


def float_layers(raw_layers, blas: bool = False) -> list:
    """Checkpoint layers -> FloatLayers (T_r[x] and A_r precomputed in float64). blas: the routed layers' tables as
    one batched matrix product (the same products summed in another order: last-bit differences from the default,
    whose bits the export's goldens record; for timing runs on large random models)."""
    out = []
    for i, p in enumerate(raw_layers):
        if blas and i > 0:
            table = np.matmul(p["token_embed"], np.swapaxes(p["input_proj"], 1, 2)) + p["bias"][:, None]
        else:
            table = np.einsum("lkr,vr->lvk", p["input_proj"], p["token_embed"]) + p["bias"][:, None]
        if i == 0:
            ar = np.arange(table.shape[1])
            table = table[ar, ar]                     # the token layer reads only T_x[x]
        A = transitions(p["rotation"], p["decay"]) if "rotation" in p else None
        out.append(FloatLayer(token_layer=i == 0, table=table, transition=A, readout=p["readout"],
                              unembed=p["unembed"], input_proj=p["input_proj"], token_embed=p["token_embed"],
                              bias=p["bias"], router_embed=p.get("router_embed"), router_weight=p.get("router_weight"),
                              router_bias=p.get("router_bias"), layer_input_down=p.get("layer_input_down"),
                              layer_input_proj=p.get("layer_input_proj")))
    return out


# ------------------------------------------------------------------------------------------------ synthetic checkpoints
@dataclasses.dataclass(frozen=True)
class FloatSpec:
    """Shape of a synthetic float checkpoint (the fields of yggdrasil/config.py Config that shape the parameters)."""
    d_state: int = 64
    block_size: int = 16
    router_depth: int = 6
    vocab: int = 256
    n_layers: int = 3
    router_token_dim: int = 16
    input_rank: int = 16
    readout_rank: int = 8
    layer_input_rank: int = 16
    router_state: bool = True


def random_checkpoint(spec: FloatSpec, seed: int, path) -> None:
    """Write a synthetic checkpoint (.npz, the key layout of yggdrasil/config.py:65-82): Gaussian parameters with
    scales that keep the recurrence stable (decays in [0.6, 1), small rotation generators)."""
    np.savez(path, **random_params(spec, seed))


def random_params(spec: FloatSpec, seed: int) -> dict:
    """The arrays random_checkpoint writes, by flat key."""
    rng = np.random.default_rng(seed)
    n, b, D, V, F, K, R, R2 = (spec.d_state, spec.block_size, spec.router_depth, spec.vocab, spec.router_token_dim,
                               spec.input_rank, spec.readout_rank, spec.layer_input_rank)
    arrs = {}
    for l in range(spec.n_layers):
        E = V if l == 0 else 2 ** D
        pre = "token_layer" if l == 0 else f"routed_layers/{l - 1}"
        p = {"token_embed": rng.normal(0, 1.0, (V, K)), "input_proj": rng.normal(0, 0.3 / math.sqrt(K), (E, n, K)),
             "bias": rng.normal(0, 0.1, (E, n)), "readout": rng.normal(0, 1 / math.sqrt(n), (E, R, n)),
             "unembed": rng.normal(0, 1 / math.sqrt(R), (V, R)),
             "rotation": rng.normal(0, 0.3, (E, n // b, b, b)),
             "decay": rng.uniform(0.6, 1.0, (E, n))}
        if l:
            p["router_embed"] = rng.normal(0, 1.0, (V, F))
            p["router_weight"] = rng.normal(0, 1 / math.sqrt(F + n), (2 ** D - 1, F + (n if spec.router_state else 0)))
            p["router_bias"] = rng.normal(0, 0.1, 2 ** D - 1)
            if R2:
                p["layer_input_down"] = rng.normal(0, 1 / math.sqrt(n), (R2, n))
                p["layer_input_proj"] = rng.normal(0, 0.3 / math.sqrt(R2), (E, n, R2))
        for k, v in p.items():
            arrs[f"{pre}/{k}"] = v.astype(np.float32)
    arrs["output_bias"] = rng.normal(0, 0.1, V).astype(np.float32)
    return arrs


# ------------------------------------------------------------------------------------------------ the GPU model
def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class FloatYggdrasil:
    """A float checkpoint on one GPU: the step/state API of yggdrasil/inference.py:142-202 over the float kernel."""

    def __init__(self, layers, output_bias, device=None, precision: int = 32):
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("backend='hip' needs a ROCm GPU (torch.cuda.is_available() is False)")
        if precision not in (32, 64):
            raise ValueError(f"precision {precision}: 32 or 64")
        L = _lib.lib()
        self.device = torch.device("cuda", torch.cuda.current_device() if device is None else
                                   torch.device(device).index or 0)
        self.layers_f = layers
        first = layers[0]
        self.layers, self.n = len(layers), first.n
        self.vocab, self.classes = first.token_embed.shape[0], len(output_bias)
        self.depth = layers[1].depth if len(layers) > 1 else 0
        self.precision = precision
        self.dtype = torch.float32 if precision == 32 else torch.float64
        R = first.readout.shape[1]
        R2 = layers[1].layer_input_down.shape[0] if len(layers) > 1 and layers[1].layer_input_down is not None else 0
        self.stats_stride = 3 + self.n // 16 + R
        d = _lib.FloatDesc()
        keep = []

        def arr(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a, np.float64)
            keep.append(a)
            return a.ctypes.data

        d.n_layers, d.d_state, d.block_size = self.layers, self.n, (first.transition.shape[-1] if first.transition
                                                                     is not None else 16)
        d.vocab, d.classes, d.router_depth, d.readout_rank, d.layer_input_rank = self.vocab, self.classes, self.depth, \
            R, R2
        d.router_token_dim = layers[1].router_token_dim if len(layers) > 1 else 0
        d.router_state = int(len(layers) > 1 and layers[1].routes_on_state)
        d.output_bias = arr(output_bias)
        for i, y in enumerate(layers):
            z = d.layers[i]
            z.table, z.transition, z.readout, z.unembed = arr(y.table), arr(y.transition), arr(y.readout), \
                arr(y.unembed)
            if i:
                z.router_embed, z.router_weight, z.router_bias = arr(y.router_embed), arr(y.router_weight), \
                    arr(y.router_bias)
                if R2:
                    z.layer_input_down, z.layer_input_proj = arr(y.layer_input_down), arr(y.layer_input_proj)
        h = ctypes.c_void_p()
        check(L.ygg_float_load(ctypes.byref(d), precision, self.device.index, ctypes.byref(h)))
        self._h = h
        self.output_bias = np.asarray(output_bias, np.float64)
        # the build ygg_float_run launches (csrc/ygg_float.hip: f32 builds of their own for the reference's trained
        # shapes (n, R, R2) at block 16, else the general one), as profilers name it
        shape = (self.n, R, R2)
        if precision == 32 and d.block_size == 16 and shape in ((64, 8, 16), (128, 16, 32), (256, 32, 64)):
            self.kernel_name = "ygg::float_kernel<float, %d, %d, %d, 16>" % shape
        else:
            self.kernel_name = "ygg::float_kernel<%s>" % ("float" if precision == 32 else "double")

    @classmethod
    def load(cls, path, backend: str = "hip", precision: int = 32, **kw):
        """From a float checkpoint (.npz). precision 32 (serving) or 64."""
        if backend != "hip":
            raise ValueError(f"backend {backend!r}: hip")
        if not Path(path).exists():
            raise FileNotFoundError(path)
        raw, output_bias = read(path)
        return cls(float_layers(raw), output_bias, precision=precision, **kw)

    def close(self):
        if getattr(self, "_h", None):
            _lib.lib().ygg_float_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def init_state(self, batch_size: int):
        """Zero state of batch_size streams, (B, layers, n) on the GPU."""
        import torch
        return torch.zeros(batch_size, self.layers, self.n, dtype=self.dtype, device=self.device)

    def _tokens(self, tokens):
        from .inference import device_tokens
        return device_tokens(tokens, self.vocab, self.device)

    def run(self, tokens, state=None, logits: bool = True, leaves: bool = False, stats: bool = False) -> dict:
        """T tokens per stream in one launch: tokens (B, T) -> dict(state, logits (B, T, classes), leaves (B, T, L),
        stats (L, 3 + n/16 + R) float64 maxima for calibration)."""
        import torch
        x = self._tokens(tokens)
        if x.dim() != 2:
            raise ValueError("tokens must be (B, T)")
        B, T = x.shape
        st = self.init_state(B) if state is None else state.to(self.dtype).contiguous().clone()
        if tuple(st.shape) != (B, self.layers, self.n):
            raise ValueError(f"state must be {(B, self.layers, self.n)}")
        lg = torch.empty(B, T, self.classes, dtype=self.dtype, device=self.device) if logits else None
        lv = torch.empty(B, T, self.layers, dtype=torch.int32, device=self.device) if leaves else None
        sv = torch.zeros(self.layers, self.stats_stride, dtype=torch.float64, device=self.device) if stats else None
        check(_lib.lib().ygg_float_run(self._h, _ptr(x), B, T, _ptr(st), _ptr(lg), _ptr(lv), _ptr(sv), _stream()))
        e = ctypes.c_uint32()
        out = {"state": st}
        for k, v in (("logits", lg), ("leaves", lv), ("stats", sv)):
            if v is not None:
                out[k] = v
        if stats:
            check(_lib.lib().ygg_float_take_errors(self._h, _stream(), ctypes.byref(e)))
            if e.value:
                raise YggError(6, "token out of range")
        return out

    def step(self, tokens, state):
        """One token per stream: tokens (B,) -> logits (B, classes), new state."""
        x = self._tokens(tokens)
        r = self.run(x[:, None], state)
        return r["logits"][:, 0], r["state"]

    def score(self, tokens, state=None, batch: int = 1024) -> np.ndarray:
        """Bits of tokens[:, 1:] given the tokens before them, per row of tokens (B, L), float64 (B,)."""
        import torch
        tokens = np.atleast_2d(np.asarray(tokens, np.int64))
        out = []
        for i in range(0, len(tokens), batch):
            x = tokens[i:i + batch]
            st = None if state is None else state[i:i + len(x)]
            lg = self.run(x[:, :-1], st)["logits"].double()
            y = torch.as_tensor(x[:, 1:], device=self.device)
            nll = -torch.log_softmax(lg, -1).gather(-1, y[..., None])[..., 0].sum(-1)
            out.append((nll / LN2).cpu().numpy())
        return np.concatenate(out) if out else np.zeros(0)

    def generate(self, prompt, n: int, temperature: float = 1.0, top_k: int = 0, seed: int = 0):
        """Prompt (L,) or (B, L), L >= 1, followed by n sampled tokens (yggdrasil/inference_triton.py:229-248)."""
        import torch
        prompt = np.asarray(prompt, np.int64)
        x = self._tokens(np.atleast_2d(prompt))
        r = self.run(x)
        state, logits = r["state"], r["logits"][:, -1]
        gen = torch.Generator(self.device).manual_seed(seed)
        out = [x.long()]
        for i in range(n):
            if temperature == 0:
                tok = logits.argmax(-1)
            else:
                lg = logits.float()
                if top_k:
                    lg = lg.masked_fill(lg < lg.topk(top_k, -1).values[:, -1:], -float("inf"))
                tok = torch.multinomial(torch.softmax(lg / temperature, -1), 1, generator=gen)[:, 0]
            out.append(tok[:, None])
            if i + 1 < n:
                logits, state = self.step(tok, state)
        res = torch.cat(out, 1).cpu().numpy()
        return res[0] if prompt.ndim == 1 else res


__all__ = ["FloatYggdrasil", "FloatLayer", "FloatSpec", "float_layers", "from_params", "random_checkpoint",
           "random_params", "read", "transitions"]
