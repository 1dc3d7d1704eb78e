"""Yggdrasil int8 inference on the GPU: the reference's step/state API over the int8 model file.

    model = Yggdrasil.load("model.bin")              # backend="hip": the fused gfx950 step (libygg_hip.so)
    state = model.init_state(batch_size)            # (B, layers, n) int8 on the GPU, zero
    logits, state = model.step(tokens, state)       # tokens (B,) -> logits (B, classes) f32, new state
    bits = model.score(windows)                     # (B, L) -> bits of windows[:, 1:] per window (B,) f64
    text = model.generate(prompt, 200, temperature=0.8, top_k=20)

This mirrors ``Yggdrasil`` in yggdrasil/inference.py:142-202 and ``TritonYggdrasil`` in
yggdrasil/inference_triton.py:123-248 (same method names, argument meaning, functional state and error behaviour),
but loads the int8 ``model.bin`` of cpu/export.py instead of a float checkpoint, and its state is the int8 state of
cpu/ygg.cpp (State.q, cpu/ygg.cpp:439). Steps run through the C-ABI of include/ygg_hip.h on the caller's current
torch stream; torch only provides device memory and streams.
"""
from __future__ import annotations

import ctypes
import math
import os
from pathlib import Path
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import YggError, YggInfo, check

LN2 = math.log(2.0)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def device_tokens(tokens, vocab: int, device, check_device: bool = False) -> torch.Tensor:
    """tokens as a contiguous int32 tensor on device, without waiting for the GPU. Tokens given on the host (arrays,
    lists, CPU tensors) are checked against [0, vocab) there (ValueError, as the reference rejects a bad token file up
    front, cpu/ygg.cpp:493-495) and copied through pinned memory, stream-ordered. Tokens already on the GPU are not
    read back, which would wait for every launch before them: a kernel stops a stream at a token outside [0, vocab)
    and sets bit 0 of the model's error word (take_errors()). check_device (or YGG_CHECK_TOKENS=1) checks GPU tokens
    too, at the cost of that wait."""
    if isinstance(tokens, torch.Tensor) and tokens.device.type == "cuda":
        x = tokens.to(device=device, dtype=torch.int32).contiguous()
        if (check_device or os.environ.get("YGG_CHECK_TOKENS") == "1") and x.numel() and \
                (int(x.min()) < 0 or int(x.max()) >= vocab):
            raise ValueError(f"token out of range [0, {vocab})")
        return x
    a = tokens.numpy() if isinstance(tokens, torch.Tensor) else np.asarray(tokens)
    if a.dtype.kind not in "iu":
        raise ValueError(f"tokens must be integers, got {a.dtype}")
    if a.size and (a.min() < 0 or a.max() >= vocab):
        raise ValueError(f"token out of range [0, {vocab})")
    host = torch.from_numpy(np.ascontiguousarray(a, np.int32))
    if host.numel():
        host = host.pin_memory()
    return host.to(device, non_blocking=True)


def softmax(logits: torch.Tensor, out: Optional[torch.Tensor] = None, lse: bool = True):
    """The f32 softmax the reference's time mode applies to every token's logits (cpu/ygg.cpp:59-72, 545-553), on
    the GPU (ygg_softmax): logits (..., V) f32 on a ROCm device, V <= 256 -> (probabilities of the same shape, equal to
    the reference's to the bit, in out if given (it may be logits itself); the log-sum-exp of each row, (...) f32, or
    None when lse is False). Stream-ordered on the current stream; nothing waits."""
    if not (isinstance(logits, torch.Tensor) and logits.device.type == "cuda" and logits.dtype == torch.float32):
        raise ValueError("logits must be a float32 tensor on a ROCm device")
    if logits.dim() < 1:
        raise ValueError("logits need a class axis")
    V = logits.shape[-1]
    if not 1 <= V <= 256:
        raise ValueError(f"V = {V} outside [1, 256]")
    x = logits.contiguous()
    p = torch.empty_like(x) if out is None else out
    if p.shape != x.shape or p.dtype != torch.float32 or not p.is_contiguous() or p.device != x.device:
        raise ValueError("out must be a contiguous float32 tensor shaped like logits, on the same device")
    ls = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device) if lse else None
    with torch.cuda.device(x.device):
        check(_lib.lib().ygg_softmax(_ptr(x), x.numel() // V if V else 0, V, _ptr(p), _ptr(ls), _stream()))
    return p, ls


class Yggdrasil:
    """An int8 model on one GPU (the ``hip`` backend)."""

    softmax = staticmethod(softmax)

    def __init__(self, path, device=None, graph: bool = False, check_tokens: bool = False):
        if not torch.cuda.is_available():
            raise RuntimeError("backend='hip' needs a ROCm GPU (torch.cuda.is_available() is False)")
        L = _lib.lib()
        self.device = torch.device("cuda", torch.cuda.current_device() if device is None else
                                   torch.device(device).index or 0)
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            check(L.ygg_load(str(path).encode(), self.device.index, ctypes.byref(h)))
        self._h = h
        info = YggInfo()
        check(L.ygg_model_info(h, ctypes.byref(info)))
        self.info = info
        self.layers, self.n, self.vocab = info.n_layers, info.d_state, info.vocab
        self.classes, self.depth = info.vocab, info.router_depth
        self.graph = graph
        self.check_tokens = check_tokens
        self._graphs = {}

    @classmethod
    def load(cls, path, backend: str = "hip", **kw):
        """From an int8 model file (YGG1, cpu/export.py). backend "hip": the fused gfx950 step; kw device, graph
        (replay one captured step per batch size, as the Triton backend's cuda_graph), check_tokens (also range-check
        tokens that are already on the GPU, which waits for the stream). A float checkpoint (.npz) loads
        the float step instead (yggdrasil_amd.float_model.FloatYggdrasil; kw device, precision 32 or 64)."""
        if backend != "hip":
            raise ValueError(f"backend {backend!r}: hip")
        if not Path(path).exists():
            raise FileNotFoundError(path)
        if str(path).endswith(".npz"):
            from .float_model import FloatYggdrasil
            return FloatYggdrasil.load(path, backend=backend, **kw)
        try:
            _lib.lib()
        except ImportError as e:
            raise ImportError(f"backend='hip' needs the built library ({e})") from e
        return cls(path, **kw)

    def kernel_name(self, B: int, T: int, generate: bool = False, score: bool = False) -> str:
        """The kernel a call of B streams and T tokens launches (generate: `generate` of T tokens; score: `score`, or
        `run` with a digest), by the name profilers show for it."""
        if generate and score:
            raise ValueError("generate and score are different calls")
        buf = ctypes.create_string_buffer(128)
        check(_lib.lib().ygg_kernel_name(self._h, B, T, 1 if generate else (2 if score else 0), buf, len(buf)))
        return buf.value.decode()

    def spec_stats(self, reset: bool = False) -> dict:
        """Counters of generation with speculating helpers (one stream): steps taken from a helper's slot, steps the
        stream computed itself, helper wavefronts that served a step, that started, that stopped waiting. Waits for
        the device."""
        import torch
        torch.cuda.synchronize(self.device)
        out = (ctypes.c_uint64 * 5)()
        _lib.check(_lib.lib().ygg_spec_stats(self._h, out, int(reset)))
        return dict(zip(("hits", "misses", "helpers_served", "helpers_started", "helpers_timed_out"), list(out)))

    def close(self):
        if getattr(self, "_h", None):
            self._graphs.clear()
            _lib.lib().ygg_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------------------------------------------ state
    def init_state(self, batch_size: int) -> torch.Tensor:
        """Zero state of batch_size streams, (B, layers, n) int8 on the GPU."""
        return torch.zeros(batch_size, self.layers, self.n, dtype=torch.int8, device=self.device)

    def _tokens(self, tokens, shape=None) -> torch.Tensor:
        x = device_tokens(tokens, self.vocab, self.device, self.check_tokens)
        if shape is not None and tuple(x.shape) != tuple(shape):
            raise ValueError(f"tokens of shape {tuple(x.shape)}, expected {tuple(shape)}")
        return x

    def _check_state(self, state: torch.Tensor, B: int) -> torch.Tensor:
        if state.dtype != torch.int8 or tuple(state.shape) != (B, self.layers, self.n):
            raise ValueError(f"state must be int8 {(B, self.layers, self.n)}, got {state.dtype} {tuple(state.shape)}")
        if state.device != self.device:
            raise ValueError(f"state on {state.device}, model on {self.device}")
        return state.contiguous()

    # ------------------------------------------------------------------------------------------------ step
    def _step(self, x: torch.Tensor, state: torch.Tensor):
        B = x.shape[0]
        logits = torch.empty(B, self.vocab, dtype=torch.float32, device=self.device)
        out = torch.empty_like(state)
        check(_lib.lib().ygg_step(self._h, _ptr(x), _ptr(state), _ptr(out), _ptr(logits), None, B, _stream()))
        return logits, out

    def step(self, tokens, state: torch.Tensor):
        """One token per stream: tokens (B,) -> logits (B, classes) of the next token, new state (B, layers, n)."""
        x = self._tokens(tokens)
        if x.dim() != 1:
            raise ValueError("tokens must be (B,)")
        state = self._check_state(state, x.shape[0])
        if not self.graph:
            return self._step(x, state)
        B = x.shape[0]
        if B not in self._graphs:
            sx = torch.zeros(B, dtype=torch.int32, device=self.device)
            sh = self.init_state(B)
            self._step(sx, sh)
            torch.cuda.synchronize(self.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                out = self._step(sx, sh)
            self._graphs[B] = g, sx, sh, out
        g, sx, sh, (logits, h) = self._graphs[B]
        sx.copy_(x)
        sh.copy_(state)
        g.replay()
        return logits.clone(), h.clone()

    def run(self, tokens, state: Optional[torch.Tensor] = None, logits: bool = True, leaves: bool = False,
            states: bool = False, digest=False, _entry: str = "ygg_run") -> dict:
        """T tokens per stream in one launch: tokens (B, T) from state (default zero; not modified) ->
        dict(state=(B, layers, n) after the last token, logits=(B, T, classes), leaves=(B, T, layers) int32,
        states=(B, T, layers, n) int8, digest=(B,) int64 bit pattern of the uint64 digest).

        Tokens given on the host are range-checked before the launch (ValueError). Tokens already on the GPU are not
        read back: a stream whose token t lies outside [0, vocab) stops there, its state stays the one before token
        t, and its rows of logits, leaves and states from token t on are left unwritten (the uninitialised memory of
        this call's outputs); take_errors() returns bit 0 for it. So with GPU tokens that may be out of range, call
        take_errors() (or pass them through device_tokens(..., check_device=True)) before trusting the outputs."""
        x = self._tokens(tokens)
        if x.dim() != 2:
            raise ValueError("tokens must be (B, T)")
        B, T = x.shape
        st = self.init_state(B) if state is None else self._check_state(state, B).clone()
        dev = self.device
        out = {"state": st}
        lg = torch.empty(B, T, self.vocab, dtype=torch.float32, device=dev) if logits else None
        lv = torch.empty(B, T, self.layers, dtype=torch.int32, device=dev) if leaves else None
        sv = torch.empty(B, T, self.layers, self.n, dtype=torch.int8, device=dev) if states else None
        if isinstance(digest, torch.Tensor):
            dg = digest.to(device=dev, dtype=torch.int64).clone()
        elif digest:
            dg = torch.full((B,), np.int64(np.uint64(0xCBF29CE484222325).view(np.int64)), dtype=torch.int64,
                            device=dev)
        else:
            dg = None
        check(getattr(_lib.lib(), _entry)(self._h, _ptr(x), B, T, _ptr(st), _ptr(lg), _ptr(lv), _ptr(sv), _ptr(dg),
                                          _stream()))
        for k, v in (("logits", lg), ("leaves", lv), ("states", sv), ("digest", dg)):
            if v is not None:
                out[k] = v
        return out

    def run_grouped(self, tokens, state: Optional[torch.Tensor] = None, logits: bool = True, leaves: bool = False,
                    states: bool = False, digest=False) -> dict:
        """run() computed leaf-grouped (ygg_run_grouped): the streams that take the same expert at a (token, layer) are
        updated together, on int8 MFMA for large groups. Same arguments and results as run()."""
        return self.run(tokens, state, logits, leaves, states, digest, _entry="ygg_run_grouped")

    def take_errors(self) -> int:
        """Wait for the current stream; the error bits kernels set since the last call (bit 0: bad token)."""
        e = ctypes.c_uint32()
        check(_lib.lib().ygg_take_errors(self._h, _stream(), ctypes.byref(e)))
        return e.value

    # ------------------------------------------------------------------------------------------------ consumers
    @torch.no_grad()
    def score(self, tokens, state: Optional[torch.Tensor] = None, batch: int = 1024, targets=None) -> np.ndarray:
        """Bits of tokens[:, 1:] given the tokens before them, per row of tokens (B, L), as float64 (B,); with
        targets (B, L), bits of targets[:, t] given tokens[:, :t + 1] (every token an input, as the reference scores
        windows x against their next tokens y). Rows start from state, or from zero (yggdrasil/inference.py:179-188).
        One fused launch per batch of rows: the step and the float64 log-softmax of the reference's score mode
        (cpu/ygg.cpp:513-516), no logits written."""
        tokens = np.atleast_2d(np.asarray(tokens, np.int64))
        if targets is not None:
            targets = np.atleast_2d(np.asarray(targets, np.int64))
            if targets.shape != tokens.shape:
                raise ValueError(f"targets {targets.shape} for tokens {tokens.shape}")
        out = []
        for i in range(0, len(tokens), batch):
            rows = tokens[i:i + batch]
            if targets is None:
                xin, tgt = rows[:, :-1], rows[:, 1:]
            else:
                xin, tgt = rows, targets[i:i + batch]
            B, T = xin.shape
            st = self.init_state(B) if state is None else self._check_state(state[i:i + B], B).clone()
            nll = torch.zeros(B, dtype=torch.float64, device=self.device)
            if T > 0:
                xd, yd = self._tokens(np.ascontiguousarray(xin)), self._tokens(np.ascontiguousarray(tgt))
                check(_lib.lib().ygg_score(self._h, _ptr(xd), _ptr(yd), B, T, _ptr(st), _ptr(nll), _stream()))
            out.append((nll / LN2).cpu().numpy())
        return np.concatenate(out) if out else np.zeros(0)

    @torch.no_grad()
    def generate(self, prompt, n: int, temperature: float = 1.0, top_k: int = 0, seed: int = 0,
                 return_logits: bool = False):
        """Prompt (L,) or (B, L), L >= 1, followed by n sampled tokens. temperature 0: greedy
        (yggdrasil/inference.py:190-202, yggdrasil/inference_triton.py:229-248). The prompt but its last token goes
        through one ygg_run launch; the n sampled tokens come from one ygg_generate launch that samples on the device
        and feeds each token back as the next input. Draws depend on (seed, row, position) only, so a row samples the
        same tokens whatever the batch around it. return_logits: also the logits (B, n, classes) each token was
        sampled from."""
        prompt = np.asarray(prompt, np.int64)
        if prompt.ndim not in (1, 2) or prompt.shape[-1] < 1:
            raise ValueError("prompt must be (L,) or (B, L) with L >= 1")
        if n < 0:
            raise ValueError(f"n = {n} < 0")
        if not (temperature >= 0 and math.isfinite(temperature)):
            raise ValueError(f"temperature {temperature}: finite and >= 0")
        if top_k < 0:
            raise ValueError(f"top_k {top_k} < 0")
        x = self._tokens(np.atleast_2d(prompt))
        B = x.shape[0]
        st = self.run(x[:, :-1], logits=False)["state"] if x.shape[1] > 1 else self.init_state(B)
        toks = torch.empty(B, n, dtype=torch.int32, device=self.device)
        lg = torch.empty(B, n, self.vocab, dtype=torch.float32, device=self.device) if return_logits else None
        first = x[:, -1].contiguous()
        check(_lib.lib().ygg_generate(self._h, _ptr(first), B, n, _ptr(st), ctypes.c_float(temperature), int(top_k),
                                      ctypes.c_uint64(seed & (2 ** 64 - 1)), _ptr(toks), _ptr(lg), _stream()))
        res = torch.cat([x, toks], 1).long().cpu().numpy()
        res = res[0] if prompt.ndim == 1 else res
        return (res, lg) if return_logits else res


def load(path, backend: str = "hip", **kw) -> Yggdrasil:
    return Yggdrasil.load(path, backend=backend, **kw)


__all__ = ["Yggdrasil", "YggError", "load"]
