"""Build the gfx950 library (libygg_hip.so, in this package directory) and, for the tests, the CPU oracle.

    python -m yggdrasil_amd.build            # the HIP library
    python -m yggdrasil_amd.build --oracle   # also oracle/libygg_oracle.so and, where /root/reference exists,
                                             # the reference kernel in oracle/_ref/

The library is built in-tree so that it travels with the source tree; objects go to _build/ (git-ignored).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libygg_hip.so"
BUILD = PKG / "_build"
ORACLE = ROOT / "oracle"
REFERENCE_CPU = Path("/root/reference/cpu")

ARCH = "gfx950"
# -ffp-contract=off: every f32 multiply and add rounds separately, as the reference (cpu/Makefile:5).
# packed-fp32-ops off: no v_pk_* f32 instructions are generated.
HIPCC_FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-ffp-contract=off", "-fPIC",
               "-mcode-object-version=5", "-Wall", "-Wno-unused-result",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
SOURCES = ["ygg_kernels.hip", "ygg_kernels_fast.hip", "ygg_kernels_fast_x.hip", "ygg_kernels_fact.hip",
           "ygg_kernels_deep.hip", "ygg_kernels_flow.hip", "ygg_kernels_group.hip",
           "ygg_softmax.hip", "ygg_capi.hip", "ygg_float.hip"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found")


def _run(cmd, cwd=None):
    r = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"{' '.join(map(str, cmd))} failed:\n{r.stdout}\n{r.stderr}")
    return r


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link libygg_hip.so (always rebuilds)."""
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []

    def compile_one(src):
        obj = BUILD / (Path(src).stem + ".o")
        _run([cc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
        return obj
    with cf.ThreadPoolExecutor(len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_oracle(verbose: bool = False) -> None:
    """The C oracle, and the reference kernel where its source is present (test infrastructure)."""
    _run(["make", "-s", "-C", str(ORACLE), "-B", "libygg_oracle.so"])
    if (REFERENCE_CPU / "ygg.cpp").exists():
        _run(["make", "-s", "-C", str(ORACLE), "-B", "ref", f"REF={REFERENCE_CPU}"])
    if verbose:
        print(f"built {ORACLE / 'libygg_oracle.so'}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--oracle", action="store_true")
    a = ap.parse_args()
    build_library(verbose=True)
    if a.oracle:
        build_oracle(verbose=True)


if __name__ == "__main__":
    main()
