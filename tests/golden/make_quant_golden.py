"""Write tests/golden/quant_golden.npz: the reference's int8 quantisation (cpu/export.py:216-265, `quantize`) of a
synthetic float model, the expected output for yggdrasil_amd.export.quantize.

Run in the build container, where /root/reference exists:

    python tests/golden/make_quant_golden.py

The float model is yggdrasil_amd.float_model.random_checkpoint(SPEC, SEED) (deterministic; a sha256 of its float64
arrays is recorded so that a drifting generator is caught), its FloatLayers come from yggdrasil_amd.float_model, and
the calibration maxima from the float64 restatement oracle/float_oracle.py over seeded token windows (recorded as
inputs). The reference's `quantize` is imported from /root/reference/cpu/export.py and called on those same arrays,
wrapped in its own FloatLayer/LayerStats dataclasses; its outputs (integer arrays and float32 scales) are recorded
for three settings: tensor scales at margin 1.0, group scales at margin 0.85, factored storage at margin 0.7 (the
transitions and layer-input projections, which no setting changes, for the first only). Only numbers are recorded:
inputs (the stats), outputs and hashes.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import float_oracle as FO  # noqa: E402
from yggdrasil_amd import float_model as FM  # noqa: E402

OUT = Path(__file__).resolve().parent / "quant_golden.npz"
SPEC = FM.FloatSpec(d_state=64, block_size=16, router_depth=3, vocab=16, n_layers=3, router_token_dim=8,
                    input_rank=8, readout_rank=8, layer_input_rank=16)
SEED = 5
SETTINGS = [("tensor_1.0", 1.0, False, False), ("group_0.85", 0.85, True, False), ("factored_0.7", 0.7, False, True)]
FIELDS = ("transition", "readout", "readout_scale", "unembed", "unembed_scale", "table", "router_weight",
          "router_threshold", "rms_eps", "state_r2", "layer_input_down", "layer_input_down_scale", "layer_input_proj",
          "layer_input_scale")
FACTORED_FIELDS = ("input_proj", "input_scale", "bias", "token_code", "token_scale")


def model(tmp: Path):
    p = tmp / "float.npz"
    FM.random_checkpoint(SPEC, SEED, p)
    raw, ob = FM.read(p)
    return FM.float_layers(raw), ob


def layers_digest(layers) -> str:
    h = hashlib.sha256()
    for fl in layers:
        for k in ("table", "transition", "readout", "unembed", "input_proj", "token_embed", "bias", "router_embed",
                  "router_weight", "router_bias", "layer_input_down", "layer_input_proj"):
            v = getattr(fl, k)
            if v is not None:
                h.update(np.ascontiguousarray(v, np.float64).tobytes())
    return h.hexdigest()


def calib_tokens():
    return np.random.default_rng(11).integers(0, SPEC.vocab, (16, 48))


def small(v):
    """Integer arrays stored in the narrowest of int16/int32 that holds them (values are compared, not types)."""
    v = np.asarray(v)
    if v.dtype.kind in "iu" and v.size:
        for t in (np.int16, np.int32):
            if v.min() >= np.iinfo(t).min and v.max() <= np.iinfo(t).max:
                return v.astype(t)
    return v


SHARED = ("transition", "layer_input_proj")   # the same in every setting: recorded for the first only


def flatten(quant, prefix: str, first: bool) -> dict:
    out = {}
    for l, q in enumerate(quant):
        for k in FIELDS:
            v = getattr(q, k)
            if v is not None and (first or k not in SHARED):
                out[f"{prefix}/{l}/{k}"] = small(v)
        if q.factored is not None:
            for k in FACTORED_FIELDS:
                out[f"{prefix}/{l}/factored_{k}"] = small(getattr(q.factored, k))
    return out


def main():
    import tempfile
    sys.path.insert(0, "/root/reference")
    sys.path.insert(0, "/root/reference/cpu")
    import export as RE                    # the reference cpu/export.py (float model helpers need no JAX)
    with tempfile.TemporaryDirectory() as tmp:
        layers, ob = model(Path(tmp))
    stats = FO.run(layers, ob, calib_tokens())["stats"]
    n = SPEC.d_state
    g = n // 16
    ref_layers = []
    for fl in layers:
        table = fl.table
        if fl.token_layer:                 # the reference's token-layer table is (V, V, n); quantize reads T_x[x]
            V = table.shape[0]
            full = np.zeros((V, V, n))
            full[np.arange(V), np.arange(V)] = table
            table = full
        ref_layers.append(RE.FloatLayer(
            token_layer=fl.token_layer, transition=fl.transition, table=table, input_proj=fl.input_proj,
            token_embed=fl.token_embed, bias=fl.bias, readout=fl.readout, unembed=fl.unembed,
            router_embed=fl.router_embed, router_weight=fl.router_weight, router_bias=fl.router_bias,
            layer_input_down=fl.layer_input_down, layer_input_proj=fl.layer_input_proj, depth=fl.depth))
    ref_stats = [RE.LayerStats(float(r[0]), float(r[1]), float(r[2]), np.array(r[3:3 + g]), np.array(r[3 + g:]))
                 for r in stats]
    rec = {"stats": stats, "layers_sha256": np.array(layers_digest(layers))}
    for i, (name, hm, group, fac) in enumerate(SETTINGS):
        rec.update(flatten(RE.quantize(ref_layers, ref_stats, hm, group, fac), name, i == 0))
    np.savez_compressed(OUT, **rec)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(rec)} arrays)")


if __name__ == "__main__":
    main()
