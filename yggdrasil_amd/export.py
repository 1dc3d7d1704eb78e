"""int8 export of a float checkpoint: calibration, quantisation and the YGG1 file, with the GPU in both loops.

    x, y = windows(train_tokens, 256, 128)                  # consecutive windows and their next tokens
    rec = export("run.npz", "model.bin", x, y)

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
SCALE_FLOOR = 1e-12                # no quantisation range is taken below this
STATE_GROUP = 16                   # state coordinates that share one scale under group scales
GROUP_SCALE_FLOOR = 1e-3           # under group scales no group range is below this fraction of the widest
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


# ------------------------------------------------------------------------------------------------- quantisation
# Every float64 expression below that feeds an int8 code or an f32 scale of the file is evaluated in the operation
# order the reference's quantiser uses (cpu/export.py:158-171, 216-265), so that the written file is the one the
# reference writes from the same float model and maxima; the list of these expressions is part of this build's
# design notes.

def symmetric(w: np.ndarray, per_row: bool):
    """Symmetric int8 codes of w and their scale: range = max |w| over the last axis (per_row, one scale per row) or
    over all of w, floored at SCALE_FLOOR; scale = range / 127; codes = rint(w / scale) as int64."""
    rng = np.abs(w).max(-1) if per_row else np.abs(w).max()
    scale = np.maximum(rng, SCALE_FLOOR) / INT8_MAX
    return np.rint(w / (scale[..., None] if per_row else scale)).astype(np.int64), scale


def saturate16(x: np.ndarray) -> np.ndarray:
    """rint, saturated to the int16 range, as int16."""
    return np.clip(np.rint(x), -32768, 32767).astype(np.int16)


@dataclasses.dataclass(frozen=True)
class StateScale:
    """The float value of one int8 unit of a layer's state: per coordinate (unit, (n,)) and the largest of them
    (ref), the unit the layer's single scales are stated in. The layer above reads this state through rms(), so it
    sees each coordinate at unit / ref relative to ref."""
    unit: np.ndarray
    ref: float

    @property
    def relative(self) -> np.ndarray:
        return self.unit / self.ref

    @staticmethod
    def of(st: LayerStats, n: int, hmargin: float, group: bool) -> "StateScale":
        """One unit for the whole state (the state maximum times hmargin over 127), or, under group scales, one
        per STATE_GROUP coordinates from the group maxima, each floored at GROUP_SCALE_FLOOR of the widest."""
        if not group:
            ref = st.state_max * hmargin / INT8_MAX
            return StateScale(np.full(n, ref), ref)
        gmax = np.asarray(st.state_group_max, np.float64)
        floor = GROUP_SCALE_FLOOR * max(np.max(st.state_group_max), SCALE_FLOOR)
        per_group = np.maximum(gmax, floor) * hmargin / INT8_MAX
        return StateScale(np.repeat(per_group, STATE_GROUP), float(per_group.max()))


def _readout_unembed(fl, st: LayerStats, own: StateScale, group: bool) -> dict:
    """P and Q with their scales. The readout z = P_r h is quantised at max|z| / 127; P is per tensor with the state
    unit in its scalar scale, or, under group scales, per row with the state units folded into the rows first; Q is
    per tensor or per class, its scale times z's unit."""
    z_unit = max(st.readout_max, SCALE_FLOOR) / INT8_MAX
    if group:
        P, p_scale = symmetric(fl.readout * own.unit[None, None, :], per_row=True)
        readout_scale = (p_scale / z_unit).astype(f32)
    else:
        P, p_scale = symmetric(fl.readout, per_row=False)
        readout_scale = f32(p_scale * own.ref / z_unit)
    Q, q_scale = symmetric(fl.unembed, per_row=group)
    return dict(readout=P, readout_scale=readout_scale, unembed=Q, unembed_scale=f32(q_scale * z_unit))


def _inputs(fl, own: StateScale, factored: bool) -> dict:
    """The token's input in state units: a table row per (expert, token) (the token layer keeps each expert's own
    token row only), or the factored form T_r[x] = rint(f32(U_r v[x]) f32(su_r mT)) + c_r with U_r per expert,
    v per tensor and c_r, mT in state units."""
    if fl.token_layer:
        return dict(table=saturate16(fl.table / own.unit)[:, None])
    if not factored:
        table = np.empty(fl.table.shape, np.int16)
        for j in range(0, len(fl.table), 256):            # in slices of experts, to bound the float64 temporaries
            table[j:j + 256] = saturate16(fl.table[j:j + 256] / own.unit)
        return dict(table=table)
    E = len(fl.input_proj)
    codes, proj_scale = symmetric(fl.input_proj.reshape(E, -1), per_row=True)
    token_codes, token_scale = symmetric(fl.token_embed, per_row=False)
    return dict(factored=Factored(input_proj=codes.reshape(fl.input_proj.shape), input_scale=proj_scale.astype(f32),
                                  bias=saturate16(fl.bias / own.unit), token_code=token_codes,
                                  token_scale=(token_scale / own.unit).astype(f32)))


def _router(fl, below: StateScale, group: bool) -> dict:
    """Node tests of a routed layer on the int8 state below, read at below.ref: per-row int8 weights of the state
    part (its coordinates rescaled to below.ref first), and the token part folded into a per-(token, node)
    threshold in units of the row's scale; rms_eps in below.ref units; under group scales the squared relative
    group scales of the state below, for its sum of squares."""
    F = fl.router_token_dim
    token_part = fl.router_embed @ fl.router_weight[:, :F].T + fl.router_bias[None, :]      # (V, nodes)
    w, w_scale = symmetric(fl.router_weight[:, F:] * below.relative[None, :], per_row=True)
    out = dict(router_weight=w, router_threshold=(-token_part / w_scale[None, :]).astype(f32),
               rms_eps=f32(RMS_EPS / below.ref ** 2))
    if group:
        out["state_r2"] = (below.relative[::STATE_GROUP] ** 2).astype(f32)
    return out


def _layer_input(fl, st: LayerStats, own: StateScale, below: StateScale, group: bool) -> dict:
    """The routed layer's input from the layer below, zl = V' rms(h_below) at max|zl| / 127 with V' per row on the
    state below (rescaled to below.ref), then U'_r zl per tensor, added in this layer's state units (per coordinate
    under group scales)."""
    if fl.layer_input_down is None:
        return {}
    down, down_scale = symmetric(fl.layer_input_down * below.relative[None, :], per_row=True)
    zl_unit = max(st.layer_input_max, SCALE_FLOOR) / INT8_MAX
    proj, proj_scale = symmetric(fl.layer_input_proj, per_row=False)
    scale = proj_scale * zl_unit / own.unit
    return dict(layer_input_down=down, layer_input_down_scale=(down_scale / zl_unit).astype(f32),
                layer_input_proj=proj, layer_input_scale=scale.astype(f32) if group else f32(scale[0]))


def quantize(layers, stats: Sequence[LayerStats], hmargin: float = 1.0, group: bool = False,
             factored: bool = False) -> list:
    """Int8 QuantLayers of float64 FloatLayers from their calibration maxima: one state scale per layer, or one per
    16 coordinates (group); hmargin scales the state ranges; factored stores the routed inputs factored instead of
    as tables (the reference's scheme, cpu/export.py:216-265)."""
    out, below = [], None
    for fl, st in zip(layers, stats):
        own = StateScale.of(st, fl.n, hmargin, group)
        parts = dict(token_layer=fl.token_layer, n=fl.n, block=fl.transition.shape[-1], depth=fl.depth,
                     transition=np.rint(fl.transition * 2.0 ** SHIFT).astype(np.int64))
        parts.update(_readout_unembed(fl, st, own, group))
        parts.update(_inputs(fl, own, factored))
        if not fl.token_layer:
            parts.update(_router(fl, below, group))
            parts.update(_layer_input(fl, st, own, below, group))
        out.append(QuantLayer(**parts))
        below = own
    return out


def windows(ids, seq_len: int, m: int):
    """Consecutive next-token windows of one token stream: up to m windows x (m, seq_len) and their targets y, the
    token after each of x's (the window pairing of tasks/text.py:28-32 that the reference calibrates and scores
    on)."""
    ids = np.asarray(ids)
    m = min(m, (len(ids) - 1) // seq_len)
    run = np.asarray(ids[:m * seq_len + 1], np.int64)
    return run[:-1].reshape(m, seq_len), run[1:].reshape(m, seq_len)


def int8_bits(quant, output_bias, x: np.ndarray, y: np.ndarray, router_token_dim: int, input_rank: int) -> float:
    """Bits per prediction of y (S, T) given x (S, T) under the int8 model `quant`, every window from the zero
    state, scored on the GPU in one fused launch per 1024 windows (the reference scores int_forward's logits of x
    against y, cpu/export.py:554-561)."""
    from .inference import Yggdrasil
    with tempfile.TemporaryDirectory() as tmp:
        p = Path(tmp) / "cand.bin"
        write(quant, output_bias, p, router_token_dim=router_token_dim, input_rank=input_rank)
        m = Yggdrasil.load(p)
        try:
            bits = m.score(x, targets=y)
        finally:
            m.close()
    return float(bits.sum() / y.size)


def export(npz, out, x: np.ndarray, y: np.ndarray = None, hmargin: float = 0.0, storage: str = "table",
           state_scale: str = "auto") -> dict:
    """Calibrate on the windows x (S, T), quantize, write out (YGG1) and out.json; returns the export record
    (cpu/export.py:531-558). y (S, T) are the targets of x (windows()); without y, x holds (S, T + 1) windows whose
    first T tokens are the inputs and last T the targets. The calibration maxima come from the inputs only; the
    candidates are compared by bits per target. hmargin 0 picks from HMARGIN_GRID, state_scale "auto" picks tensor or
    group scales, both by those bits."""
    import torch
    t0 = time.time()
    x = np.ascontiguousarray(x, np.int64)
    if y is None:
        if x.ndim != 2 or x.shape[1] < 2:
            raise ValueError("windows without targets must be (S, T + 1) with T >= 1")
        x, y = np.ascontiguousarray(x[:, :-1]), np.ascontiguousarray(x[:, 1:])
    y = np.ascontiguousarray(y, np.int64)
    if x.shape != y.shape or x.ndim != 2:
        raise ValueError(f"inputs {x.shape} and targets {y.shape}: both (S, T)")
    raw, output_bias = read(npz)
    layers = float_layers(raw)
    for i, fl in enumerate(layers):
        if fl.transition is None:
            raise NotImplementedError("experts without transitions have no int8 export")
        if i and not fl.routes_on_state:
            raise NotImplementedError("routing on the token only has no int8 export")
    m64 = FloatYggdrasil(layers, output_bias, precision=64)
    try:
        stats = calibrate(m64, x)
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
            cal[(mode, hm)] = int8_bits(q, output_bias, x, y, F, K)
    mode, hm = min(cal, key=cal.get)
    args = dict(hmargin=hm, group=mode == "group", factored=fac)
    hdr, nbytes = write(quantize(layers, stats, **args), output_bias, out, router_token_dim=F, input_rank=K)
    res = dict(header=hdr, bytes=nbytes, quantize=args, state_scale=mode, storage=storage,
               calib_windows=int(x.shape[0]), calib_seq_len=int(x.shape[1]),
               calib_bpc={f"{k[0]}_{k[1]}": v for k, v in cal.items()},
               stats=[{k: (v.tolist() if isinstance(v, np.ndarray) else v) for k, v in dataclasses.asdict(s).items()}
                      for s in stats],
               secs=round(time.time() - t0, 1))
    Path(str(out) + ".json").write_text(json.dumps(res))
    return res


__all__ = ["LayerStats", "calibrate", "quantize", "export", "int8_bits", "stats_from_array", "windows"]
