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

def header(layers: Sequence[QuantLayer], vocab: int, router_token_dim: int = 0, input_rank: int = 0) -> dict:
    """HEADER values of layers, checked against LIMITS; ValueError names the failing field (cpu/export.py:353-379)."""
    q0, routed = layers[0], list(layers[1:])
    R2 = routed[0].layer_input_proj.shape[2] if routed and routed[0].layer_input_proj is not None else 0
    fac = [q.factored for q in layers if q.factored is not None]
    hdr = dict(n_layers=len(layers), d_state=q0.n, block_size=q0.block, vocab=vocab,
               router_depth=routed[0].depth if routed else 0, readout_rank=q0.readout.shape[1],
               layer_input_rank=R2, reserved=0, router_token_dim=router_token_dim,
               input_rank=fac[0].input_proj.shape[2] if fac else input_rank, shift=SHIFT)

    def need(ok, field):
        if not ok:
            raise ValueError(f"model.bin cannot hold {field} = {hdr.get(field)} (limits {LIMITS})")
    for k in ("d_state", "block_size", "readout_rank"):
        need(hdr[k] in LIMITS[k], k)
    need(R2 % RANK_MULTIPLE == 0 and R2 <= LIMITS["max_layer_input_rank"], "layer_input_rank")
    need(vocab <= LIMITS["max_vocab"], "vocab")
    need(1 <= len(layers) <= LIMITS["max_layers"], "n_layers")
    need(not routed or 1 <= hdr["router_depth"] <= LIMITS["max_router_depth"], "router_depth")
    need(not fac or (hdr["input_rank"] % RANK_MULTIPLE == 0
                     and RANK_MULTIPLE <= hdr["input_rank"] <= LIMITS["max_input_rank"]), "input_rank")
    for q in routed:
        need(q.depth == hdr["router_depth"], "router_depth")
        need(q.readout.shape[1] == hdr["readout_rank"], "readout_rank")
        need((q.layer_input_proj is not None) == bool(R2) and (not R2 or q.layer_input_proj.shape[2] == R2),
             "layer_input_rank")
    return hdr


# ----------------------------------------------------------------------------------------------------- writer

ArraySource = Union[np.ndarray, "Streamed"]


@dataclasses.dataclass
class Streamed:
    """An array written in chunks (the expert records of a large model): nbytes and an iterator of byte chunks."""
    nbytes: int
    chunks: Callable[[], Iterator[np.ndarray]]


def layer_arrays(l: int, q: QuantLayer, hdr: dict, record_chunk: int = 0) -> list:
    """(name, array) of layer l in file order (the order of cpu/export.py:382-441).

    record_chunk > 0 streams the expert records in chunks of that many experts instead of building them at once."""
    n, V, R, R2 = hdr["d_state"], hdr["vocab"], hdr["readout_rank"], hdr["layer_input_rank"]
    VP, tag, arrs = round_up(V, CLASS_PAD), f"l{l}_", []

    def add(name, a):
        arrs.append((tag + name, a if isinstance(a, Streamed) else np.ascontiguousarray(a)))
    if not q.token_layer:
        E = 2 ** q.depth
        thr = np.zeros((V, E), f32)        # heap order from node 1: slot 0 unused
        thr[:, 1:] = q.router_threshold
        add("thr", thr)
        if q.state_r2 is not None:
            add("r2b", np.asarray(q.state_r2, f32))
        if np.ndim(q.layer_input_scale):
            add("mulv", np.asarray(q.layer_input_scale, f32))
        if q.factored is not None:
            add("vt", np.asarray(q.factored.token_code).astype(np.int8))
            add("mT", np.asarray(q.factored.token_scale, f32))
        w = np.zeros((E, n), np.int64)
        w[1:] = q.router_weight
        add("w", (w + 128).astype(np.uint8))
        if R2:
            add("vl", pack_layer_input_down(q.layer_input_down, n))
            mv = np.zeros(round_up(R2, 16), f32)
            mv[:R2] = q.layer_input_down_scale
            add("mv", mv)
    E = len(q.transition)
    sizes = {"transition": 2 * n * q.block}
    if not q.token_layer and R2:
        sizes["layer_input_proj"] = n * R2
    sizes["readout"] = R * n
    if q.factored is not None:
        k = q.factored.input_proj.shape[2]
        sizes.update(input_proj=n * k, bias=2 * n, input_scale=4)
    else:
        sizes["table"] = q.table.shape[1] * n * 2
    offset, off = {k: -1 for k in RECORD}, 0
    for k, s in sizes.items():
        offset[k] = off
        off += s
    record_bytes = round_up(off, ALIGN)

    def records(j0, j1):
        rec = np.zeros((j1 - j0, record_bytes), np.uint8)
        parts = {"transition": pack_transition(q.transition[j0:j1])}
        if "layer_input_proj" in sizes:
            parts["layer_input_proj"] = pack_proj(q.layer_input_proj[j0:j1])
        parts["readout"] = pack_readout(q.readout[j0:j1])
        if q.factored is not None:
            fc = q.factored
            parts["input_proj"] = pack_proj(fc.input_proj[j0:j1])
            parts["bias"] = np.ascontiguousarray(np.asarray(fc.bias[j0:j1], "<i2")).view(np.uint8)
            parts["input_scale"] = np.ascontiguousarray(np.asarray(fc.input_scale[j0:j1], f32)[:, None]).view(np.uint8)
        else:
            parts["table"] = np.ascontiguousarray(np.asarray(q.table[j0:j1], "<i2")).reshape(j1 - j0, -1).view(np.uint8)
        for k, a in parts.items():
            rec[:, offset[k]:offset[k] + sizes[k]] = a
        return rec
    meta = [record_bytes] + [offset[k] for k in RECORD]
    add("meta", np.array(meta if q.factored is not None else meta[:-FACTORED_PARTS], np.int32))
    if record_chunk and E > record_chunk:
        add("rec", Streamed(E * record_bytes,
                            lambda: (records(j, min(E, j + record_chunk)) for j in range(0, E, record_chunk))))
    else:
        add("rec", records(0, E))
    add("Q", pack_unembed(q.unembed, VP))
    if np.ndim(q.unembed_scale):
        sv = np.zeros(VP, f32)
        sv[:V] = q.unembed_scale
        add("sqv", sv)
    if np.ndim(q.readout_scale):           # R = 8: kernel lane i holds row i / 2
        add("mzl", np.repeat(np.asarray(q.readout_scale, f32), 2, axis=1) if R == 8
            else np.asarray(q.readout_scale, f32))
    scal = dict(readout_scale=q.readout_scale, unembed_scale=q.unembed_scale, rms_eps=q.rms_eps,
                layer_input_scale=q.layer_input_scale)
    add("scal", np.array([0 if v is None or np.ndim(v) else v for v in (scal[k] for k in SCALARS)], f32))
    return arrs


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
