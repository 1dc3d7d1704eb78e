"""The C-ABI library on any host: it is built for gfx950, loads, exports every entry point include/ygg_hip.h declares,
and reports bad arguments and malformed model files with YGG_* codes before touching a device (the reference dies
with exit 1 on the same files, cpu/ygg.cpp:41-43, 137-202). No kernel is launched here."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from yggdrasil_amd import fmt, synth

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ygg_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(ygg_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from yggdrasil_amd import _lib
    return _lib


def test_library_built_for_gfx950():
    so = ROOT / "yggdrasil_amd" / "libygg_hip.so"
    assert so.exists(), "run python -m yggdrasil_amd.build"
    out = subprocess.run(["/opt/rocm/llvm/bin/clang-offload-bundler", "--list", "--type=o", f"--input={so}"],
                         capture_output=True, text=True)
    if out.returncode == 0 and out.stdout.strip():
        assert "gfx950" in out.stdout
    else:   # the bundle sits in a .hip_fatbin section; the target id appears in it
        assert b"gfx950" in so.read_bytes()


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert set(names) == set(lib.SYMBOLS), names
    L = lib.lib()
    for n in names:
        assert hasattr(L, n), n
    nm = subprocess.run(["nm", "-D", "--defined-only", str(lib.LIB_PATH)], capture_output=True, text=True).stdout
    for n in names:
        assert re.search(rf"\bT {n}$", nm, flags=re.M), n


def test_version_and_info_layout(lib):
    L = lib.lib()
    assert L.ygg_version() == lib.ABI_VERSION
    # ygg_info: 22 int32 + 2 int64 + 8 int64
    assert ctypes.sizeof(lib.YggInfo) == 22 * 4 + 8 * 10
    assert lib.YggInfo.file_array_bytes.offset == 22 * 4


def test_bad_arguments(lib):
    L = lib.lib()
    h = ctypes.c_void_p()
    assert L.ygg_load(None, 0, ctypes.byref(h)) == 5
    assert L.ygg_load(b"/x", 0, None) == 5
    assert L.ygg_load_blob(None, 10, 0, ctypes.byref(h)) == 5
    assert L.ygg_model_info(None, None) == 5
    assert L.ygg_run(None, None, 1, 1, None, None, None, None, None, None) == 5
    assert L.ygg_run_grouped(None, None, 1, 1, None, None, None, None, None, None) == 5
    assert L.ygg_run_grouped_noalloc(None, None, 1, 1, None, None, None, None, None, None) == 5
    assert L.ygg_step(None, None, None, None, None, None, 1, None) == 5
    assert L.ygg_take_errors(None, None, None) == 5
    assert L.ygg_generate(None, None, 1, 1, None, 0.0, 0, 0, None, None, None) == 5
    assert L.ygg_kernel_name(None, 1, 1, 0, ctypes.create_string_buffer(8), 8) == 5
    assert L.ygg_float_load(None, 32, 0, ctypes.byref(h)) == 5
    assert L.ygg_float_run(None, None, 1, 1, None, None, None, None, None) == 5
    d = lib.FloatDesc()
    assert L.ygg_float_load(ctypes.byref(d), 16, 0, ctypes.byref(h)) == 5      # precision
    d.n_layers, d.d_state, d.block_size, d.vocab, d.classes, d.readout_rank = 2, 72, 8, 16, 16, 8
    assert L.ygg_float_load(ctypes.byref(d), 32, 0, ctypes.byref(h)) == 3      # d_state not a multiple of 16
    assert b"unsupported shape" in L.ygg_last_error()
    # a missing array is reported before any device is touched
    d.d_state, d.router_depth, d.router_token_dim, d.router_state = 64, 2, 4, 1
    assert L.ygg_float_load(ctypes.byref(d), 32, 0, ctypes.byref(h)) == 5
    assert b"output_bias is NULL" in L.ygg_last_error()
    ob = np.zeros(16)
    d.output_bias = ob.ctypes.data
    assert L.ygg_float_load(ctypes.byref(d), 64, 0, ctypes.byref(h)) == 5
    assert b"layer 0 lacks an array" in L.ygg_last_error() and not h.value
    L.ygg_float_free(None)
    assert L.ygg_load(b"/nonexistent/model.bin", 0, ctypes.byref(h)) == 1
    assert b"cannot open" in L.ygg_last_error()
    L.ygg_free(None)


def test_malformed_files(lib, tmp_path):
    L = lib.lib()
    good = tmp_path / "good.bin"
    synth.write_model(synth.KERNEL_CASES[3], 1, good)
    data = good.read_bytes()
    i = data.find(b"l1_w\0")
    bad = {
        "magic": (b"XGG1" + data[4:], 2, b"not a model file"),
        "truncated": (data[:len(data) // 2], 2, b"short model file"),
        "d_state": (data[:8] + np.int32(72).tobytes() + data[12:], 3, b"LIMITS"),
        "missing": (data[:i] + b"l1_X" + data[i + 4:], 2, b"missing l1_w"),
        # an entry whose offset + bytes overflows int64 must not pass the bounds check
        "overflow": (data[:52 + 32] + np.int64(1 << 62).tobytes() + np.int64(1 << 62).tobytes() + data[52 + 48:], 2,
                     b"short model file (array"),
    }
    h = ctypes.c_void_p()
    for name, (blob, code, msg) in bad.items():
        p = tmp_path / f"{name}.bin"
        p.write_bytes(blob)
        assert L.ygg_load(str(p).encode(), 0, ctypes.byref(h)) == code, name
        assert msg in L.ygg_last_error(), (name, L.ygg_last_error())
        assert not h.value
    # scales that are not finite (a NaN readout scale, an infinite output bias, a NaN layer-input row scale)
    arr = np.frombuffer(data, np.uint8)
    mf = fmt.parse(arr)

    def at(name, k, value):
        off = mf.arrays[name].__array_interface__["data"][0] - arr.__array_interface__["data"][0] + 4 * k
        return data[:off] + np.float32(value).tobytes() + data[off + 4:]
    for name, k, value in (("l1_scal", 0, np.nan), ("head_b", 3, np.inf), ("l1_scal", 2, -np.nan),
                           ("l0_scal", 1, -np.inf)):
        p = tmp_path / f"nonfinite_{name}.bin"
        p.write_bytes(at(name, k, value))
        assert L.ygg_load(str(p).encode(), 0, ctypes.byref(h)) == 2, name
        assert b"not finite" in L.ygg_last_error(), (name, L.ygg_last_error())
        assert not h.value
    # a well-formed file gets as far as the device: YGG_ERR_DEVICE without one
    rc = L.ygg_load(str(good).encode(), 0, ctypes.byref(h))
    import torch
    if not torch.cuda.is_available():
        assert rc == 7 and b"no HIP device" in L.ygg_last_error()
    else:
        assert rc == 0
        L.ygg_free(h)


def test_host_api_errors(tmp_path):
    from yggdrasil_amd.inference import Yggdrasil
    with pytest.raises(ValueError, match="backend"):
        Yggdrasil.load("model.bin", backend="jax")
    with pytest.raises(FileNotFoundError):
        Yggdrasil.load(tmp_path / "none.bin")
