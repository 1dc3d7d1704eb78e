"""TEST INFRASTRUCTURE ONLY: Python access to the C oracle (libygg_oracle.so) and to the reference kernel binaries in
oracle/_ref/. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.

``Oracle(path).run(tokens, ...)`` restates the reference step (cpu/ygg.cpp:441-459) for B streams x T tokens from
a given int8 state; ``ref_dump`` and ``ref_logits`` run the reference kernel itself (cpu/ygg.cpp:500-525) through its
CLI and the dump driver oracle/ref_dump.cpp.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import tempfile
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libygg_oracle.so"
REF_DIR = HERE / "_ref"
REF_YGG = REF_DIR / "ygg"
REF_DUMP = REF_DIR / "ygg_dump"
REF_SOFTMAX = REF_DIR / "ygg_softmax"
DIGEST_INIT = 0xCBF29CE484222325
DIGEST_MUL = 0x100000001B3
DIGEST_LEAF = 0xD6E8FEB86659FD93
DIGEST_COORD = 0x9E3779B97F4A7C15

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise ImportError(f"{LIB} not built (make -C oracle)")
        L = ctypes.CDLL(str(LIB))
        vp = ctypes.c_void_p
        L.yo_load.argtypes = [ctypes.c_char_p, ctypes.POINTER(vp), ctypes.c_char_p, ctypes.c_int]
        L.yo_free.argtypes = [vp]
        L.yo_info.argtypes = [vp, vp]
        L.yo_run.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_char_p,
                             ctypes.c_int]
        L.yo_run_sums.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp, vp, vp, ctypes.c_int, ctypes.c_char_p,
                                  ctypes.c_int]
        L.yo_softmax.argtypes = [vp, ctypes.c_long, ctypes.c_int, vp, vp]
        _lib = L
    return _lib


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class OracleError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class Oracle:
    """The C restatement of the reference step on one model file."""

    def __init__(self, path):
        L = lib()
        h = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        rc = L.yo_load(str(path).encode(), ctypes.byref(h), err, 512)
        if rc:
            raise OracleError(rc, err.value.decode())
        self._h = h
        self._free = L.yo_free      # (kept on the instance: at interpreter exit the module's globals may be gone)
        info = np.zeros(12, np.int32)
        L.yo_info(h, _ptr(info))
        (self.n_layers, self.n, self.block, self.vocab, self.depth, self.readout_rank, self.layer_input_rank,
         self.input_rank, self.shift, self.n_experts, self.vocab_pad, factored) = (int(v) for v in info)
        self.factored = bool(factored)

    def close(self):
        if getattr(self, "_h", None):
            self._free(self._h)
            self._h = None

    __del__ = close

    def run(self, tokens, state=None, logits=True, leaves=True, states=False, digest=False, threads=None):
        """tokens (B, T) -> dict with the final state (B, L, n) and, as asked, logits (B, T, V), leaves (B, T, L),
        states (B, T, L, n) and digest (B,) uint64 (continuing from digest when it is an array)."""
        x = np.ascontiguousarray(tokens, np.int32)
        B, T = x.shape
        L, n, V = self.n_layers, self.n, self.vocab
        st = np.zeros((B, L, n), np.int8) if state is None else np.array(state, np.int8, copy=True, order="C")
        out = {"state": st}
        lg = np.empty((B, T, V), np.float32) if logits else None
        lv = np.empty((B, T, L), np.int32) if leaves else None
        sv = np.empty((B, T, L, n), np.int8) if states else None
        if isinstance(digest, np.ndarray):
            dg = np.array(digest, np.uint64, copy=True)
        else:
            dg = np.full(B, DIGEST_INIT, np.uint64) if digest else None
        err = ctypes.create_string_buffer(512)
        th = threads or min(os.cpu_count() or 1, 16, max(B, 1))
        rc = lib().yo_run(self._h, _ptr(x), B, T, _ptr(st), _ptr(lg), _ptr(lv), _ptr(sv), _ptr(dg), th, err, 512)
        if rc:
            raise OracleError(rc, err.value.decode())
        for k, v in (("logits", lg), ("leaves", lv), ("states", sv), ("digest", dg)):
            if v is not None:
                out[k] = v
        return out


    def run_sums(self, tokens, state=None, threads=None):
        """tokens (B, T) -> (digest (B,) uint64, lgsum (B,) uint64, final state): the digest of every leaf and state,
        and the sum of the f32 bit patterns (as uint32) of every logit, per stream; nothing per token is kept, so it
        runs at any size."""
        x = np.ascontiguousarray(tokens, np.int32)
        B, T = x.shape
        st = np.zeros((B, self.n_layers, self.n), np.int8) if state is None else \
            np.array(state, np.int8, copy=True, order="C")
        dg = np.full(B, DIGEST_INIT, np.uint64)
        ls = np.zeros(B, np.uint64)
        err = ctypes.create_string_buffer(512)
        th = threads or min(os.cpu_count() or 1, 16, max(B, 1))
        rc = lib().yo_run_sums(self._h, _ptr(x), B, T, _ptr(st), _ptr(dg), _ptr(ls), th, err, 512)
        if rc:
            raise OracleError(rc, err.value.decode())
        return dg, ls, st


def softmax(logits: np.ndarray):
    """The f32 softmax of the reference's `time` mode (cpu/ygg.cpp:44-72) over the last axis of logits: (probs of the
    same shape, log-sum-exp of each row)."""
    lg = np.ascontiguousarray(logits, np.float32)
    V = lg.shape[-1]
    rows = lg.size // V if V else 0
    pr = np.empty_like(lg)
    ls = np.empty(lg.shape[:-1], np.float32)
    if rows:
        lib().yo_softmax(_ptr(lg), rows, V, _ptr(pr), _ptr(ls))
    return pr, ls


def logit_bits_sum(logits: np.ndarray) -> np.ndarray:
    """Per stream, the sum of the f32 bit patterns (as uint32) of logits (B, T, V), as uint64."""
    b = np.ascontiguousarray(logits, np.float32).view(np.uint32).astype(np.uint64)
    return b.reshape(b.shape[0], -1).sum(-1, dtype=np.uint64)


def digest_of(leaves: np.ndarray, states: np.ndarray, init=None) -> np.ndarray:
    """The per-stream digest of leaves (B, T, L) and states (B, T, L, n), computed in NumPy (uint64 wrap-around)."""
    B, T, L = leaves.shape
    n = states.shape[-1]
    coord = ((2 * np.arange(n, dtype=np.uint64) + np.uint64(1)) * np.uint64(DIGEST_COORD))
    d = np.full(B, DIGEST_INIT if init is None else init, np.uint64)
    with np.errstate(over="ignore"):
        for t in range(T):
            for l in range(L):
                f = leaves[:, t, l].astype(np.uint32).astype(np.uint64) * np.uint64(DIGEST_LEAF)
                f = f + ((states[:, t, l].view(np.uint8).astype(np.uint64) + np.uint64(1)) * coord).sum(-1,
                                                                                                        dtype=np.uint64)
                d = d * np.uint64(DIGEST_MUL) + f + np.uint64(l)
    return d


_M64 = (1 << 64) - 1


def mix64(z: int) -> int:
    """SplitMix64's output function (Steele, Lea, Flood, "Fast splittable pseudorandom number generators", 2014) on
    the state after one increment: the first output of splitmix64 seeded z."""
    z = (z + 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def sample_uniform(seed: int, b: int, t: int) -> float:
    """The uniform in [0, 1) that ygg_generate draws for stream b at step t: the top 24 bits of
    mix64(seed ^ mix64(b << 32 | t)) / 2^24."""
    r = mix64((seed & _M64) ^ mix64(((b << 32) | t) & _M64))
    return (r >> 40) / float(1 << 24)


def sample(logits: np.ndarray, temperature: float, top_k: int, u: float):
    """The class ygg_generate takes from the logits (V,) of one step given its uniform u, in float64: temperature 0
    -> the first maximal class (argmax, yggdrasil/inference.py:102-104); else classes below the top_k-th largest logit
    are dropped (yggdrasil/inference.py:105-106) and the first class whose running sum of exp((lg - max) / temperature)
    exceeds u times the total is taken (inverse CDF). Returns (class, margin): margin is the distance of u times the
    total to the nearest running sum, relative to the total; a float32 implementation may differ where it is tiny."""
    lg = np.asarray(logits, np.float64)
    if temperature == 0:
        return int(np.argmax(lg)), 1.0
    keep = np.ones(lg.shape, bool)
    if 0 < top_k < lg.size:
        keep = lg >= np.sort(lg)[-top_k]
    w = np.where(keep, np.exp((lg - lg.max()) / temperature), 0.0)
    cdf = np.cumsum(w)
    target = u * cdf[-1]
    idx = np.nonzero((cdf > target) & (w > 0))[0]
    c = int(idx[0]) if idx.size else int(np.nonzero(w > 0)[0][-1])
    return c, float(np.min(np.abs(cdf[w > 0] - target)) / cdf[-1])


def have_ref() -> bool:
    return REF_YGG.exists() and REF_DUMP.exists()


def ref_dump(model_path, tokens: np.ndarray):
    """Run the reference kernel's dump driver: tokens (B, T), zero state per stream -> logits, leaves, states."""
    x = np.ascontiguousarray(tokens, np.int32)
    B, T = x.shape
    with tempfile.TemporaryDirectory() as tmp:
        xf, lf, vf, sf = (os.path.join(tmp, f) for f in ("x.i32", "lg.f32", "lv.i32", "st.i8"))
        x.tofile(xf)
        subprocess.run([str(REF_DUMP), str(model_path), xf, str(B), str(T), lf, vf, sf], check=True,
                       stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)
        lg = np.fromfile(lf, np.float32)
        lv = np.fromfile(vf, np.int32)
        sv = np.fromfile(sf, np.int8)
    L = lv.size // (B * T)
    return dict(logits=lg.reshape(B, T, -1), leaves=lv.reshape(B, T, L), states=sv.reshape(B, T, L, -1))


def have_ref_softmax() -> bool:
    return REF_SOFTMAX.exists()


def ref_softmax(logits: np.ndarray):
    """The reference's own softmax() (cpu/ygg.cpp:59-72) through oracle/_ref/ygg_softmax: (probs, lse) per row."""
    lg = np.ascontiguousarray(logits, np.float32)
    V = lg.shape[-1]
    rows = lg.size // V
    with tempfile.TemporaryDirectory() as tmp:
        lf, pf, sf = (os.path.join(tmp, f) for f in ("lg.f32", "p.f32", "s.f32"))
        lg.tofile(lf)
        subprocess.run([str(REF_SOFTMAX), str(rows), str(V), lf, pf, sf], check=True, stdout=subprocess.DEVNULL,
                       stderr=subprocess.PIPE)
        return np.fromfile(pf, np.float32).reshape(lg.shape), np.fromfile(sf, np.float32).reshape(lg.shape[:-1])


def ref_logits(model_path, tokens: np.ndarray) -> np.ndarray:
    """`ygg logits` of the reference kernel (cpu/ygg.cpp:500-525): tokens (B, T) -> logits (B, T, V)."""
    x = np.ascontiguousarray(tokens, np.int32)
    B, T = x.shape
    with tempfile.TemporaryDirectory() as tmp:
        xf, of = os.path.join(tmp, "x.i32"), os.path.join(tmp, "o.f32")
        x.tofile(xf)
        subprocess.run([str(REF_YGG), "logits", str(model_path), xf, str(B), str(T), of], check=True,
                       stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)
        return np.fromfile(of, np.float32).reshape(B, T, -1)


def ref_time(model_path, tokens_1d: np.ndarray, seg: int = 2000, warm: int = 1000, cpu: Optional[int] = None) -> str:
    """`ygg time` of the reference kernel (cpu/ygg.cpp:528-562) on one stream; returns its output line."""
    with tempfile.TemporaryDirectory() as tmp:
        xf = os.path.join(tmp, "x.i32")
        np.ascontiguousarray(tokens_1d, np.int32).tofile(xf)
        cmd = [str(REF_YGG), "time", str(model_path), xf, "--seg", str(seg), "--warm", str(warm)]
        if cpu is not None:
            cmd = ["taskset", "-c", str(cpu)] + cmd
        return subprocess.run(cmd, check=True, capture_output=True, text=True).stdout.strip()


def ref_score(model_path, x: np.ndarray, y: np.ndarray) -> float:
    """`ygg score` of the reference kernel (cpu/ygg.cpp:500-519): bits per token of targets y given inputs x (B, T),
    zero state per row, as the printed bpc (6 decimals)."""
    x = np.ascontiguousarray(x, np.int32)
    y = np.ascontiguousarray(y, np.int32)
    B, T = x.shape
    with tempfile.TemporaryDirectory() as tmp:
        xf, yf = os.path.join(tmp, "x.i32"), os.path.join(tmp, "y.i32")
        x.tofile(xf)
        y.tofile(yf)
        out = subprocess.run([str(REF_YGG), "score", str(model_path), xf, yf, str(B), str(T)], check=True,
                             capture_output=True, text=True).stdout
    return float(out.split("bpc=")[1].split()[0])


def nll_bits(logits: np.ndarray, targets: np.ndarray) -> np.ndarray:
    """Bits per row of targets (B, T) under logits (B, T, V), the formula of the reference's score mode
    (cpu/ygg.cpp:514-516) in float64: log(sum exp(lg - max)) + max - lg[y]."""
    lg = logits.astype(np.float64)
    mx = lg.max(-1)
    se = np.exp(lg - mx[..., None]).sum(-1)
    ly = np.take_along_axis(lg, targets[..., None].astype(np.int64), -1)[..., 0]
    return (np.log(se) + mx - ly).sum(-1) / np.log(2.0)
