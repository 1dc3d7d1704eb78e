"""YGG1 model files: the int8 weight layout of the reference's CPU kernel, read and written from logical arrays.

The container is the reference's format, unchanged (``cpu/export.py:34-51`` FORMAT, ``cpu/ygg.cpp:78-220`` reader):

    "YGG1", int32 HEADER fields, int32 array count,
    array table [(char name[32], int64 offset, int64 bytes)], padded to 64,
    the arrays, each 64-byte aligned, offsets relative to the first array.

Per layer ``l`` the arrays are ``l<l>_<tag>``; ``l<l>_meta`` holds the expert record size and the byte offsets of the
record parts (-1: absent), ``l<l>_scal`` the four scalars. Every u8 weight array stores ``w + 128``.

The logical model (``QuantLayer``) follows ``cpu/export.py:174-205``; the packers follow the layouts documented at
``cpu/export.py:321-350`` and ``cpu/export.py:382-441`` and are written here from those layout descriptions. ``d_state``
may also be 96 (the reference LIMITS allow 64, 128, 256; this build's kernels and oracle take any multiple of 16
that fits its lane mapping, see ``D_STATES``).
"""
from __future__ import annotations

import dataclasses
import struct
from pathlib import Path
from typing import Callable, Iterable, Iterator, Optional, Sequence, Union

import numpy as np

f32 = np.float32
MAGIC = b"YGG1"
HEADER = ("n_layers", "d_state", "block_size", "vocab", "router_depth", "readout_rank", "layer_input_rank",
          "reserved", "router_token_dim", "input_rank", "shift")          # cpu/export.py:41-42
RECORD = ("transition", "layer_input_proj", "readout", "table", "input_proj", "bias", "input_scale")  # :43
FACTORED_PARTS = 3
SCALARS = ("readout_scale", "unembed_scale", "rms_eps", "layer_input_scale")  # :46
OUTPUT_BIAS = "head_b"
SHIFT = 14
STATE_GROUP = 16
CLASS_PAD = 32
ALIGN = 64
RANK_MULTIPLE = 4
# The reference LIMITS (cpu/export.py:47-48) plus d_state = 96, which this build's kernels and oracle also run.
D_STATES = (64, 96, 128, 256)
LIMITS = dict(d_state=D_STATES, block_size=(8, 16), readout_rank=(8, 16, 32), max_layer_input_rank=64,
              max_input_rank=64, max_vocab=256, max_layers=8, max_router_depth=16)
REFERENCE_D_STATES = (64, 128, 256)
HEADER_STRUCT = struct.Struct("<4s12i")     # magic + 11 header fields + array count = 52 bytes
ENTRY_STRUCT = struct.Struct("<32sqq")


def round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


@dataclasses.dataclass
class Factored:
    """Factored input of a routed layer (cpu/export.py:174-181)."""
    input_proj: np.ndarray            # (E, n, k) int8 values
    input_scale: np.ndarray           # (E,) f32
    bias: np.ndarray                  # (E, n) int16
    token_code: np.ndarray            # (V, k) int8 values
    token_scale: np.ndarray           # (n,) f32


@dataclasses.dataclass
class QuantLayer:
    """One int8 layer in logical (unpacked) form (cpu/export.py:184-205). Integer arrays hold signed values."""
    token_layer: bool
    n: int
    block: int
    depth: int
    transition: np.ndarray            # (E, n/b, b, b) A16
    readout: np.ndarray               # (E, R, n)
    readout_scale: Union[np.float32, np.ndarray]   # f32, or (E, R)
    unembed: np.ndarray               # (V, R)
    unembed_scale: Union[np.float32, np.ndarray]   # f32, or (V,)
    table: Optional[np.ndarray] = None            # (E, V, n) int16; token layer (V, 1, n)
    factored: Optional[Factored] = None
    router_weight: Optional[np.ndarray] = None    # (2^D - 1, n)
    router_threshold: Optional[np.ndarray] = None  # (V, 2^D - 1) f32
    rms_eps: np.float32 = f32(0)
    state_r2: Optional[np.ndarray] = None         # (n/16,) f32
    layer_input_down: Optional[np.ndarray] = None  # (R2, n)
    layer_input_down_scale: Optional[np.ndarray] = None  # (R2,) f32
    layer_input_proj: Optional[np.ndarray] = None  # (E, n, R2)
    layer_input_scale: Union[None, np.float32, np.ndarray] = None  # f32, or (n,)


# ----------------------------------------------------------------------------------------------------- packers
# Each packer returns per-expert rows of bytes (E, bytes); the layouts are those ygg.cpp reads.

def pack_transition(A16: np.ndarray) -> np.ndarray:
    """(E, n/b, b, b) int16 values -> per expert [n/16 row groups][b/2 column pairs][16 rows][2] int16 bytes.

    Row i of the state sits in block i // b; its column pair p covers block columns 2p, 2p+1 (cpu/export.py:321-326,
    read by add_transition, cpu/ygg.cpp:311-332)."""
    E, nb, b, _ = A16.shape
    n = nb * b
    # rows in 16-row groups: (E, n/16, 16, b) -> column pairs -> (E, n/16, b/2, 16, 2)
    rows = A16.reshape(E, n, b).reshape(E, n // 16, 16, b // 2, 2)
    out = np.ascontiguousarray(np.moveaxis(rows, 3, 2).astype("<i2"))
    return out.reshape(E, -1).view(np.uint8)


def pack_proj(u: np.ndarray) -> np.ndarray:
    """(E, n, rank) signed -> per expert [rank/4][n][4] u8 (u + 128) (cpu/export.py:329-332)."""
    E, n, k = u.shape
    a = (u.astype(np.int64) + 128).astype(np.uint8).reshape(E, n, k // 4, 4)
    return np.ascontiguousarray(a.transpose(0, 2, 1, 3)).reshape(E, -1)


def pack_readout(p: np.ndarray) -> np.ndarray:
    """(E, R, n) signed -> per expert u8 (p + 128): R = 8: [n/8][16 lanes][4], lane 2r + e holding
    P[r][8c + 4e .. 8c + 4e + 3]; R >= 16: [R/16][n/4][16 rows][4] (cpu/export.py:335-342, cpu/ygg.cpp:393-420)."""
    E, R, n = p.shape
    u = (p.astype(np.int64) + 128).astype(np.uint8)
    if R >= 16:
        a = u.reshape(E, R // 16, 16, n // 4, 4).transpose(0, 1, 3, 2, 4)
    else:
        # (E, r, c, e, k) -> (E, c, r, e, k): lane = 2r + e
        a = u.reshape(E, R, n // 8, 2, 4).transpose(0, 2, 1, 3, 4)
    return np.ascontiguousarray(a).reshape(E, -1)


def pack_unembed(Q: np.ndarray, VP: int) -> np.ndarray:
    """(V, R) signed -> [R/4][VP][4] u8 (q + 128), padded classes weight 0 (cpu/export.py:345-350)."""
    V, R = Q.shape
    full = np.zeros((VP, R), np.int64)
    full[:V] = Q
    return np.ascontiguousarray((full + 128).astype(np.uint8).reshape(VP, R // 4, 4).transpose(1, 0, 2))


def pack_layer_input_down(Vd: np.ndarray, n: int) -> np.ndarray:
    """(R2, n) signed -> [RG][n/4][16][4] u8 (v + 128), rows padded to 16 RG with zeros (cpu/export.py:402-406)."""
    R2 = Vd.shape[0]
    RG = round_up(R2, 16) // 16
    full = np.zeros((16 * RG, n), np.int64)
    full[:R2] = Vd
    u = (full + 128).astype(np.uint8).reshape(RG, 16, n // 4, 4)
    return np.ascontiguousarray(u.transpose(0, 2, 1, 3))


# ----------------------------------------------------------------------------------------------------- header

def _layer_input_rank(q: QuantLayer) -> int:
    return 0 if q.layer_input_proj is None else int(q.layer_input_proj.shape[2])


def _limit_violations(hdr: dict, layers: Sequence[QuantLayer], factored: bool) -> Iterator[str]:
    """The header fields whose values a YGG1 file cannot hold, in the order they are checked. Each routed layer must
    also agree with the header, which is taken from the first one."""
    for field, allowed in (("d_state", LIMITS["d_state"]), ("block_size", LIMITS["block_size"]),
                           ("readout_rank", LIMITS["readout_rank"])):
        if hdr[field] not in allowed:
            yield field
    r2, rank = hdr["layer_input_rank"], hdr["input_rank"]
    if r2 % RANK_MULTIPLE or r2 > LIMITS["max_layer_input_rank"]:
        yield "layer_input_rank"
    if hdr["vocab"] > LIMITS["max_vocab"]:
        yield "vocab"
    if not 1 <= hdr["n_layers"] <= LIMITS["max_layers"]:
        yield "n_layers"
    if hdr["n_layers"] > 1 and not 1 <= hdr["router_depth"] <= LIMITS["max_router_depth"]:
        yield "router_depth"
    if factored and (rank % RANK_MULTIPLE or not RANK_MULTIPLE <= rank <= LIMITS["max_input_rank"]):
        yield "input_rank"
    for q in layers[1:]:
        if q.depth != hdr["router_depth"]:
            yield "router_depth"
        if q.readout.shape[1] != hdr["readout_rank"]:
            yield "readout_rank"
        if _layer_input_rank(q) != r2:
            yield "layer_input_rank"


def header(layers: Sequence[QuantLayer], vocab: int, router_token_dim: int = 0, input_rank: int = 0) -> dict:
    """The HEADER fields of a file holding layers; ValueError naming the first field outside LIMITS
    (the checks of cpu/export.py:353-379). The routed-layer fields come from the first routed layer; input_rank is
    the factored projection's rank when a layer is factored, else the value given."""
    first, routed = layers[0], layers[1:]
    fac = next((q.factored for q in layers if q.factored is not None), None)
    hdr = {"n_layers": len(layers), "d_state": first.n, "block_size": first.block, "vocab": vocab,
           "router_depth": routed[0].depth if routed else 0, "readout_rank": first.readout.shape[1],
           "layer_input_rank": _layer_input_rank(routed[0]) if routed else 0, "reserved": 0,
           "router_token_dim": router_token_dim,
           "input_rank": fac.input_proj.shape[2] if fac is not None else input_rank, "shift": SHIFT}
    bad = next(_limit_violations(hdr, layers, fac is not None), None)
    if bad is not None:
        raise ValueError(f"YGG1 header field {bad} = {hdr[bad]} is outside the format's limits {LIMITS}")
    return hdr


# ----------------------------------------------------------------------------------------------------- writer

ArraySource = Union[np.ndarray, "Streamed"]


@dataclasses.dataclass
class Streamed:
    """An array written in chunks (the expert records of a large model): nbytes and an iterator of byte chunks."""
    nbytes: int
    chunks: Callable[[], Iterator[np.ndarray]]


@dataclasses.dataclass(frozen=True)
class RecordLayout:
    """Where the parts of one expert's record lie: (part, byte offset, byte size) in record order, and the record
    size (the parts' total rounded up to ALIGN). Parts are those of RECORD; a layer has a subset of them."""
    parts: tuple
    nbytes: int

    def offset(self, part: str) -> int:
        return next((o for p, o, _ in self.parts if p == part), -1)

    def meta(self, factored: bool) -> np.ndarray:
        """l<l>_meta: the record size, then the offset of every RECORD part (-1: absent); the factored parts'
        offsets only in a factored layer."""
        tags = RECORD if factored else RECORD[:len(RECORD) - FACTORED_PARTS]
        return np.array([self.nbytes] + [self.offset(p) for p in tags], np.int32)


def record_layout(q: QuantLayer, n: int, R: int, R2: int) -> RecordLayout:
    """The record of layer q: A16 (2 bytes per entry of n/b blocks of b x b), then the routed layer-input
    projection U' (n R2 bytes), the readout P (R n bytes), and either its input table (2 n bytes per token the
    record holds a row for) or the factored projection, bias and scale."""
    sizes = [("transition", 2 * n * q.block)]
    if R2 and not q.token_layer:
        sizes.append(("layer_input_proj", n * R2))
    sizes.append(("readout", R * n))
    if q.factored is not None:
        sizes += [("input_proj", n * q.factored.input_proj.shape[2]), ("bias", 2 * n), ("input_scale", 4)]
    else:
        sizes.append(("table", 2 * n * q.table.shape[1]))
    parts, pos = [], 0
    for p, s in sizes:
        parts.append((p, pos, s))
        pos += s
    return RecordLayout(tuple(parts), round_up(pos, ALIGN))


def _part_bytes(q: QuantLayer, part: str, j0: int, j1: int) -> np.ndarray:
    """(j1 - j0, bytes) of one record part of experts j0 .. j1 - 1."""
    if part == "transition":
        return pack_transition(q.transition[j0:j1])
    if part == "layer_input_proj":
        return pack_proj(q.layer_input_proj[j0:j1])
    if part == "readout":
        return pack_readout(q.readout[j0:j1])
    if part == "table":
        return np.ascontiguousarray(np.asarray(q.table[j0:j1], "<i2")).reshape(j1 - j0, -1).view(np.uint8)
    fc = q.factored
    if part == "input_proj":
        return pack_proj(fc.input_proj[j0:j1])
    if part == "bias":
        return np.ascontiguousarray(np.asarray(fc.bias[j0:j1], "<i2")).view(np.uint8)
    return np.ascontiguousarray(np.asarray(fc.input_scale[j0:j1], f32).reshape(-1, 1)).view(np.uint8)


def pack_records(q: QuantLayer, layout: RecordLayout, j0: int, j1: int) -> np.ndarray:
    """The records of experts j0 .. j1 - 1, zero-padded to layout.nbytes each."""
    rec = np.zeros((j1 - j0, layout.nbytes), np.uint8)
    for part, off, size in layout.parts:
        rec[:, off:off + size] = _part_bytes(q, part, j0, j1)
    return rec


def _router_arrays(q: QuantLayer, n: int, V: int, R2: int) -> list:
    """(tag, array) of a routed layer ahead of its records, in file order: thresholds (V, 2^D) with the node index
    as column (column 0 belongs to no node), the optional group and factored arrays, the node weights (2^D, n) as
    u8 (w + 128, row 0 for no node) and the layer-input down-projection with its row scales (rows padded to 16)."""
    E = 2 ** q.depth
    nodes = slice(1, E)
    thr = np.zeros((V, E), f32)
    thr[:, nodes] = q.router_threshold
    out = [("thr", thr)]
    if q.state_r2 is not None:
        out.append(("r2b", np.asarray(q.state_r2, f32)))
    if np.ndim(q.layer_input_scale):
        out.append(("mulv", np.asarray(q.layer_input_scale, f32)))
    if q.factored is not None:
        out += [("vt", np.asarray(q.factored.token_code).astype(np.int8)),
                ("mT", np.asarray(q.factored.token_scale, f32))]
    weights = np.full((E, n), 128, np.uint8)
    weights[nodes] = (np.asarray(q.router_weight, np.int64) + 128).astype(np.uint8)
    out.append(("w", weights))
    if R2:
        scale = np.zeros(round_up(R2, 16), f32)
        scale[:R2] = q.layer_input_down_scale
        out += [("vl", pack_layer_input_down(q.layer_input_down, n)), ("mv", scale)]
    return out


def _readout_arrays(q: QuantLayer, V: int, R: int) -> list:
    """(tag, array) after the records, in file order: Q, the per-class unembedding scales (group scales; zero for
    padded classes), the per-(expert, row) readout scales (group scales; at R = 8 each row's scale twice, one per
    kernel lane of the row's two halves) and the four scalars (0 where an array replaces one)."""
    VP = round_up(V, CLASS_PAD)
    out = [("Q", pack_unembed(q.unembed, VP))]
    if np.ndim(q.unembed_scale):
        per_class = np.zeros(VP, f32)
        per_class[:V] = q.unembed_scale
        out.append(("sqv", per_class))
    if np.ndim(q.readout_scale):
        rows = np.asarray(q.readout_scale, f32)
        out.append(("mzl", np.repeat(rows, 2, axis=1) if R == 8 else rows))
    values = {"readout_scale": q.readout_scale, "unembed_scale": q.unembed_scale, "rms_eps": q.rms_eps,
              "layer_input_scale": q.layer_input_scale}
    out.append(("scal", np.array([0 if values[s] is None or np.ndim(values[s]) else values[s] for s in SCALARS],
                                 f32)))
    return out


def layer_arrays(l: int, q: QuantLayer, hdr: dict, record_chunk: int = 0) -> list:
    """(name, array) of layer l in file order: a routed layer's router arrays, then meta and the expert records,
    then the readout arrays (the order of cpu/export.py:382-441, which makes the file bytes the reference's).

    record_chunk > 0 streams the expert records in chunks of that many experts instead of building them at once."""
    n, V, R, R2 = hdr["d_state"], hdr["vocab"], hdr["readout_rank"], hdr["layer_input_rank"]
    layout = record_layout(q, n, R, R2)
    E = len(q.transition)
    if record_chunk and E > record_chunk:
        records = Streamed(E * layout.nbytes, lambda: (pack_records(q, layout, j, min(E, j + record_chunk))
                                                       for j in range(0, E, record_chunk)))
    else:
        records = pack_records(q, layout, 0, E)
    body = [] if q.token_layer else _router_arrays(q, n, V, R2)
    body += [("meta", layout.meta(q.factored is not None)), ("rec", records)]
    body += _readout_arrays(q, V, R)
    return [(f"l{l}_{tag}", a if isinstance(a, Streamed) else np.ascontiguousarray(a)) for tag, a in body]


def write_container(path, hdr: dict, arrs: Sequence) -> int:
    """MAGIC, header, array table, 64-byte aligned arrays -> total array bytes (cpu/export.py:444-458)."""
    tab, off = [], 0
    for name, a in arrs:
        nb = a.nbytes
        tab.append((name, off, nb))
        off += round_up(nb, ALIGN)
    with open(path, "wb") as f:
        f.write(HEADER_STRUCT.pack(MAGIC, *(hdr[k] for k in HEADER), len(arrs)))
        for name, o, nb in tab:
            if len(name.encode()) >= 32:
                raise ValueError(f"array name too long: {name}")
            f.write(ENTRY_STRUCT.pack(name.encode(), o, nb))
        f.write(b"\0" * ((-f.tell()) % ALIGN))
        for (name, a), (_, o, nb) in zip(arrs, tab):
            if isinstance(a, Streamed):
                done = 0
                for c in a.chunks():
                    f.write(c.tobytes())
                    done += c.nbytes
                if done != nb:
                    raise RuntimeError(f"{name}: streamed {done} of {nb} bytes")
            else:
                f.write(a.tobytes())
            f.write(b"\0" * (round_up(nb, ALIGN) - nb))
    return off


def write(layers: Sequence[QuantLayer], output_bias, path, router_token_dim: int = 0, input_rank: int = 0,
          record_chunk: int = 0):
    """QuantLayers -> model.bin; returns (header dict, array bytes) (cpu/export.py:461-468)."""
    V = len(output_bias)
    hdr = header(layers, V, router_token_dim, input_rank)
    ob = np.zeros(round_up(V, CLASS_PAD), f32)
    ob[:V] = output_bias
    arrs = [(OUTPUT_BIAS, ob)] + [a for l, q in enumerate(layers) for a in layer_arrays(l, q, hdr, record_chunk)]
    return hdr, write_container(path, hdr, arrs)


# ----------------------------------------------------------------------------------------------------- reader

@dataclasses.dataclass
class ModelFile:
    """A parsed YGG1 file: header fields and the raw bytes of every array (a view of one buffer)."""
    header: dict
    arrays: dict
    array_bytes: int

    def array(self, name: str, dtype) -> np.ndarray:
        return self.arrays[name].view(dtype)


def read_header(buf: Union[bytes, memoryview, np.ndarray]) -> dict:
    """Header fields of a YGG1 buffer; ValueError on a bad magic or a model outside LIMITS (cpu/ygg.cpp:137-148)."""
    mv = memoryview(buf)
    if len(mv) < HEADER_STRUCT.size:
        raise ValueError("not a model file (short header)")
    magic, *vals = HEADER_STRUCT.unpack_from(mv, 0)
    if magic != MAGIC:
        raise ValueError("not a model file (magic)")
    h = dict(zip(HEADER + ("n_arrays",), vals))
    ok = (h["d_state"] in D_STATES and h["block_size"] in (8, 16) and h["readout_rank"] in (8, 16, 32)
          and 0 <= h["layer_input_rank"] <= 64 and h["layer_input_rank"] % RANK_MULTIPLE == 0
          and 1 <= h["n_layers"] <= 8 and 1 <= h["vocab"] <= 256 and 0 <= h["router_depth"] <= 16
          and (h["n_layers"] == 1 or h["router_depth"] >= 1) and h["reserved"] == 0)
    if not ok:
        raise ValueError("unsupported model (LIMITS)")
    return h


def read(path) -> ModelFile:
    """Parse a YGG1 file into its header and named array bytes (cpu/ygg.cpp:137-171, 204-220)."""
    data = np.fromfile(path, np.uint8)
    return parse(data)


def parse(data: np.ndarray) -> ModelFile:
    h = read_header(data)
    na = h["n_arrays"]
    pos = HEADER_STRUCT.size
    end_tab = pos + na * ENTRY_STRUCT.size
    if na < 0 or len(data) < end_tab:
        raise ValueError("short array table")
    tab = [ENTRY_STRUCT.unpack_from(data, pos + i * ENTRY_STRUCT.size) for i in range(na)]
    base = round_up(end_tab, ALIGN)
    total = len(data) - base
    arrays = {}
    for name, off, nb in tab:
        key = name.rstrip(b"\0").decode()
        if off < 0 or nb < 0 or off + nb > total:
            raise ValueError(f"short model file ({key})")
        arrays[key] = data[base + off: base + off + nb]
    return ModelFile(h, arrays, total)
