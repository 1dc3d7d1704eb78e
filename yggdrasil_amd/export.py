"""int8 export of a float checkpoint: calibration, quantisation and the YGG1 file, with the GPU in both loops.

    rec = export("run.npz", "model.bin", calib_tokens)       # calib_tokens (S, T) int windows of training text

The scheme is the reference's (cpu/export.py:216-265, cpu/README.md:31-45): calibration maxima of every layer over
the calibration windows (cpu/export.py:117-153), symmetric int8 per row or per tensor, A16 = rint(2^14 A_r), tables
in units of the layer's state scale, thresholds with the token part of the router folded in. Here the maxima come from
the f64 float kernel (csrc/ygg_float.hip) instead of a JAX scan, and the margin/state-scale search scores each
candidate int8 model with the fused int8 score kernel (ygg_score) instead of the NumPy int_forward.
"""
from __future__ import annotations

import dataclasses
import json
import tempfile
import time
from pathlib import Path
from typing import Sequence

import numpy as np

from .fmt import Factored, QuantLayer, f32, write
from .float_model import FloatYggdrasil, float_layers, read

SHIFT = 14                         # A16 = rint(2^SHIFT A_r)
INT8_MAX = 127
SCALE_FLOOR = 1e-12                # smallest quantisation range
STATE_GROUP = 16                   # coordinates per state scale with group scales
GROUP_SCALE_FLOOR = 1e-3           # group scale floor, relative to the largest group
RMS_EPS = 1e-6
HMARGIN_GRID = (1.0, 0.85, 0.7, 0.6)


@dataclasses.dataclass
class LayerStats:
    """Calibration maxima of one layer (cpu/export.py:108-114)."""
    state_max: float
    layer_input_max: float
    readout_max: float
    state_group_max: np.ndarray
    readout_row_max: np.ndarray


def stats_from_array(a: np.ndarray, n: int) -> list:
    """The (L, 3 + n/16 + R) maxima of ygg_float_run -> LayerStats per layer."""
    g = n // STATE_GROUP
    return [LayerStats(float(r[0]), float(r[1]), float(r[2]), np.array(r[3:3 + g]), np.array(r[3 + g:])) for r in a]


def calibrate(model: FloatYggdrasil, windows: np.ndarray, batch: int = 4096) -> list:
    """LayerStats over windows (S, T), each from the zero state, on the model's kernel (use precision 64)."""
    import torch
    acc = None
    for i in range(0, len(windows), batch):
        s = model.run(windows[i:i + batch], logits=False, stats=True)["stats"]
        torch.cuda.synchronize()
        a = s.cpu().numpy()
        acc = a if acc is None else np.maximum(acc, a)
    return stats_from_array(acc, model.n)


def _qrow(w):
    """Symmetric int8 per row (last axis) -> (int64 values, float64 scales)."""
    s = np.maximum(np.abs(w).max(-1, keepdims=True), SCALE_FLOOR) / INT8_MAX
    return np.rint(w / s).astype(np.int64), s[..., 0]


def _qten(w):
    """Symmetric int8 per tensor -> (int64 values, scale)."""
    s = max(np.abs(w).max(), SCALE_FLOOR) / INT8_MAX
    return np.rint(w / s).astype(np.int64), s


def _sat16(x):
    return np.clip(np.rint(x), -32768, 32767)


def quantize(layers, stats: Sequence[LayerStats], hmargin: float = 1.0, group: bool = False,
             factored: bool = False) -> list:
    """Int8 QuantLayers from float64 FloatLayers and calibration stats: one state scale per layer, or one per 16
    coordinates (group) (cpu/export.py:216-265)."""
    out, rel_prev, s_prev = [], None, 1.0
    for fl, st in zip(layers, stats):
        n = fl.n
        if group:
            g = np.maximum(np.asarray(st.state_group_max, np.float64),
                           GROUP_SCALE_FLOOR * max(np.max(st.state_group_max), SCALE_FLOOR))
            sg = g * hmargin / INT8_MAX
            sc, s_ref = np.repeat(sg, STATE_GROUP), float(sg.max())
        else:
            s_ref = st.state_max * hmargin / INT8_MAX
            sc = np.full(n, s_ref)
        s_z = max(st.readout_max, SCALE_FLOOR) / INT8_MAX
        if group:          # the state scales folded into the readout rows
            readout, s_p = _qrow(fl.readout * sc[None, None, :])
            readout_scale = (s_p / s_z).astype(f32)
        else:
            readout, s_p = _qten(fl.readout)
            readout_scale = f32(s_p * s_ref / s_z)
        unembed, s_q = (_qrow if group else _qten)(fl.unembed)
        q = QuantLayer(token_layer=fl.token_layer, n=n, block=fl.transition.shape[-1], depth=fl.depth,
                       transition=np.rint(fl.transition * 2.0 ** SHIFT).astype(np.int64), readout=readout,
                       readout_scale=readout_scale, unembed=unembed, unembed_scale=f32(s_q * s_z))
        if fl.token_layer:              # one expert per token: its own row T_x[x]
            q.table = _sat16(fl.table / sc).astype(np.int16)[:, None]
        elif factored:
            vt, s_vt = _qten(fl.token_embed)
            su = np.maximum(np.abs(fl.input_proj).reshape(len(fl.input_proj), -1).max(-1), SCALE_FLOOR) / INT8_MAX
            q.factored = Factored(input_proj=np.rint(fl.input_proj / su[:, None, None]).astype(np.int64),
                                  input_scale=su.astype(f32), bias=_sat16(fl.bias / sc).astype(np.int16),
                                  token_code=vt, token_scale=(s_vt / sc).astype(f32))
        else:
            q.table = np.empty(fl.table.shape, np.int16)
            for j in range(0, len(fl.table), 256):
                q.table[j:j + 256] = _sat16(fl.table[j:j + 256] / sc)
        if not fl.token_layer:          # the layer below is quantised at s_prev * rel_prev
            F = fl.router_token_dim
            token_part = fl.router_embed @ fl.router_weight[:, :F].T + fl.router_bias[None, :]
            q.router_weight, sw = _qrow(fl.router_weight[:, F:] * rel_prev[None, :])
            q.router_threshold = (-token_part / sw[None, :]).astype(f32)
            q.rms_eps = f32(RMS_EPS / s_prev ** 2)
            if group:
                q.state_r2 = (rel_prev[::STATE_GROUP] ** 2).astype(f32)
            if fl.layer_input_down is not None:
                q.layer_input_down, sv = _qrow(fl.layer_input_down * rel_prev[None, :])
                s_v = max(st.layer_input_max, SCALE_FLOOR) / INT8_MAX
                q.layer_input_down_scale = (sv / s_v).astype(f32)
                q.layer_input_proj, s_u = _qten(fl.layer_input_proj)
                scale = s_u * s_v / sc
                q.layer_input_scale = scale.astype(f32) if group else f32(scale[0])
        rel_prev, s_prev = sc / s_ref, s_ref
        out.append(q)
    return out


def int8_bits(quant, output_bias, windows: np.ndarray, router_token_dim: int, input_rank: int) -> float:
    """Bits per token of windows[:, 1:] under the int8 model `quant`, scored on the GPU (one fused launch)."""
    from .inference import Yggdrasil
    with tempfile.TemporaryDirectory() as tmp:
        p = Path(tmp) / "cand.bin"
        write(quant, output_bias, p, router_token_dim=router_token_dim, input_rank=input_rank)
        m = Yggdrasil.load(p)
        try:
            bits = m.score(windows)
        finally:
            m.close()
    return float(bits.sum() / (windows.shape[0] * (windows.shape[1] - 1)))


def export(npz, out, calib_tokens: np.ndarray, hmargin: float = 0.0, storage: str = "table",
           state_scale: str = "auto") -> dict:
    """Calibrate on calib_tokens (S, T), quantize, write out (YGG1) and out.json; returns the export record
    (cpu/export.py:531-558). hmargin 0 picks from HMARGIN_GRID, state_scale "auto" picks tensor or group scales, both
    by the int8 model's bits per token on the calibration windows."""
    import torch
    t0 = time.time()
    raw, output_bias = read(npz)
    layers = float_layers(raw)
    for i, fl in enumerate(layers):
        if fl.transition is None:
            raise NotImplementedError("experts without transitions have no int8 export")
        if i and not fl.routes_on_state:
            raise NotImplementedError("routing on the token only has no int8 export")
    calib = np.ascontiguousarray(calib_tokens, np.int64)
    m64 = FloatYggdrasil(layers, output_bias, precision=64)
    try:
        stats = calibrate(m64, calib)
    finally:
        m64.close()
        torch.cuda.synchronize()
    fac = storage == "factored"
    F, K = layers[-1].router_token_dim, layers[0].token_embed.shape[1]
    modes = {"auto": ("tensor", "group"), "tensor": ("tensor",), "group": ("group",)}[state_scale]
    cal = {}
    for mode in modes:
        for hm in ((hmargin,) if hmargin else HMARGIN_GRID):
            q = quantize(layers, stats, hm, mode == "group", fac)
            cal[(mode, hm)] = int8_bits(q, output_bias, calib, F, K)
    mode, hm = min(cal, key=cal.get)
    args = dict(hmargin=hm, group=mode == "group", factored=fac)
    hdr, nbytes = write(quantize(layers, stats, **args), output_bias, out, router_token_dim=F, input_rank=K)
    res = dict(header=hdr, bytes=nbytes, quantize=args, state_scale=mode, storage=storage,
               calib_windows=int(calib.shape[0]), calib_seq_len=int(calib.shape[1]),
               calib_bpc={f"{k[0]}_{k[1]}": v for k, v in cal.items()},
               stats=[{k: (v.tolist() if isinstance(v, np.ndarray) else v) for k, v in dataclasses.asdict(s).items()}
                      for s in stats],
               secs=round(time.time() - t0, 1))
    Path(str(out) + ".json").write_text(json.dumps(res))
    return res


__all__ = ["LayerStats", "calibrate", "quantize", "export", "int8_bits", "stats_from_array"]
