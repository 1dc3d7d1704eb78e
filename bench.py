"""Benchmark of the int8 streaming step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 4]

Workload (default: configuration 4, the batch-4096 headline case): the synthetic V=256, 4-layer, d=128, D=14 int8 model
(3.63 GB YGG1 file, seed 3), 4096 independent streams x 1024 Zipf(1.1) byte tokens (seed 3), zero initial state.
One step = one ygg_run launch over the whole batch (every token of every stream, logits written for every token),
inputs resident in HBM before the timed region. Prints one JSON line (rank 0) with:
  value         tokens/s over the K timed steps (HIP events on the launch stream)
  roofline      compulsory HBM bytes of a launch (yggdrasil_amd.roofline, from the leaves actually taken) over the
                kernel's average duration, against 8 TB/s; traffic from the committed rocprofv3 counter summary
                when one exists for this workload
  cpu_baseline  the reference kernel (oracle/_ref/ygg `time`, built from cpu/ygg.cpp) on the host cores, one
                pinned process per core over disjoint streams, or the C oracle when the reference binary is absent
  batch1        one stream of 8192 tokens: one persistent launch, and the per-token step loop captured in hipGraphs
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import shutil
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "int8 step tokens/s @batch 4096 + % HBM roofline; batch-1 µs/token"
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_path(cfg: int, cache: Path) -> Path:
    from yggdrasil_amd import synth
    w = synth.CONFIGS[cfg]
    cache.mkdir(parents=True, exist_ok=True)
    p = cache / f"{w.name}_seed{w.model_seed}.bin"
    if not p.exists():
        t0 = time.time()
        tmp = p.with_suffix(".tmp")
        synth.write_model(w.spec, w.model_seed, tmp)
        os.replace(tmp, p)
        log(f"generated {p.name} ({p.stat().st_size / 1e9:.2f} GB) in {time.time() - t0:.1f}s")
    return p


def cpu_flags() -> set:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                return set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return set()


def cpu_baseline(path: Path, tokens: np.ndarray, procs: int, streams_per_proc: int) -> dict:
    """The reference kernel's `time` mode (cpu/ygg.cpp:528-562) on the host: `procs` processes, each pinned to one
    core, each on its own streams_per_proc streams concatenated into one token stream (state carried, f32 softmax
    per token included, as the reference times itself). Falls back to the C oracle (16 threads) when the reference
    binary is absent or the host lacks AVX-512 VNNI."""
    from oracle import oracle as O
    B, T = tokens.shape
    procs = max(1, min(procs, B // max(1, streams_per_proc)))
    ref_ok = O.REF_YGG.exists() and "avx512_vnni" in cpu_flags()
    if ref_ok:
        with tempfile.TemporaryDirectory() as tmp:
            cmds = []
            for i in range(procs):
                f = os.path.join(tmp, f"x{i}.i32")
                np.ascontiguousarray(tokens[i * streams_per_proc:(i + 1) * streams_per_proc].reshape(-1),
                                     np.int32).tofile(f)
                cmd = [str(O.REF_YGG), "time", str(path), f, "--seg", "2000", "--warm", "1000"]
                if shutil.which("taskset"):
                    cmd = ["taskset", "-c", str(i)] + cmd
                cmds.append(cmd)
            t0 = time.time()
            ps = [subprocess.Popen(c, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True) for c in cmds]
            outs = [p.communicate() for p in ps]
            wall = time.time() - t0
        if all(p.returncode == 0 for p in ps):
            med = [float(re.search(r"median=([\d.]+)", o[0]).group(1)) for o in outs]
            mean = [float(re.search(r"mean=([\d.]+)", o[0]).group(1)) for o in outs]
            thp = re.search(r"thp_kB=(-?\d+)", outs[0][0]).group(1)
            value = sum(1e9 / m for m in mean)
            ntok = streams_per_proc * T
            return {"value": round(value, 1), "unit": "tokens/s", "cores": procs, "kind": "reference",
                    "sample": f"{procs} pinned processes of `ygg time` (cpu/ygg.cpp, -O3 -march=x86-64-v4 "
                              f"-mavx512vnni), each {streams_per_proc} streams of the workload concatenated into "
                              f"{ntok} tokens (first 1000 untimed, state carried, f32 softmax per token included); "
                              f"value = sum over processes of 1e9 / mean ns/token",
                    "per_core_median_ns_per_token": round(float(np.median(med)), 1),
                    "per_core_tokens_per_s": round(1e9 / float(np.median(med)), 1),
                    "thp_kB_proc0": int(thp), "wall_s": round(wall, 1)}
        log("reference baseline failed: " + " | ".join(o[1].strip()[:200] for o in outs if o[1]))
    # the C oracle (a port), threads over streams
    n = min(B, procs * streams_per_proc)
    o = O.Oracle(path)
    x = tokens[:n]
    t0 = time.time()
    o.run(x, logits=True, leaves=False, threads=procs)
    dt = time.time() - t0
    return {"value": round(n * T / dt, 1), "unit": "tokens/s", "cores": procs, "kind": "port",
            "sample": f"C oracle (oracle/ygg_oracle.c, scalar, -O3) on {n} streams x {T} tokens, {procs} threads; "
                      f"logits only, no softmax"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=4, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--streams", type=int, default=0, help="override the configuration's stream count")
    ap.add_argument("--tokens", type=int, default=0, help="override the configuration's tokens per stream")
    ap.add_argument("--cache", default=os.environ.get("YGG_BENCH_DIR", os.path.join(tempfile.gettempdir(),
                                                                                      "ygg_bench")))
    ap.add_argument("--batch1-tokens", type=int, default=8192)
    ap.add_argument("--cpu-procs", type=int, default=16)
    ap.add_argument("--cpu-streams", type=int, default=64, help="streams per CPU baseline process")
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py runs on one GPU only: the streams are independent, so N GPUs would each run this same "
              f"workload on their own share with no communication (requested --gpus {a.gpus}).", file=sys.stderr)
        sys.exit(2)

    import torch
    from yggdrasil_amd import synth
    from yggdrasil_amd.inference import Yggdrasil
    from yggdrasil_amd.roofline import step_bytes

    w = synth.CONFIGS[a.config]
    B, T = a.streams or w.streams, a.tokens or w.steps
    path = model_path(a.config, Path(a.cache))
    t0 = time.time()
    model = Yggdrasil.load(path, device="cuda:0")
    info = model.info
    log(f"loaded {path.name} onto cuda:0 in {time.time() - t0:.1f}s: L={info.n_layers} n={info.d_state} "
        f"D={info.router_depth} V={info.vocab} device bytes {info.device_bytes / 1e9:.2f} GB")
    x_np = w.make_tokens(B, T)
    x = torch.as_tensor(x_np, device=model.device).contiguous()
    dev = model.device
    st = model.init_state(B)
    logits = torch.empty(B, T, info.vocab, dtype=torch.float32, device=dev)
    leaves = torch.empty(B, T, info.n_layers, dtype=torch.int32, device=dev)
    from yggdrasil_amd import _lib
    L = _lib.lib()
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)

    def launch(with_leaves=False):
        st.zero_()
        _lib.check(L.ygg_run(model._h, p(x), B, T, p(st), p(logits), p(leaves) if with_leaves else None, None,
                             None, sp))

    # the first warmup launch also records the leaves, for the compulsory-byte count
    for i in range(max(1, a.warmup)):
        launch(with_leaves=(i == 0))
    torch.cuda.synchronize()
    lv = leaves.cpu().numpy()
    del leaves
    alg = step_bytes(lv, x_np, info.d_state, info.block_size, info.readout_rank, info.layer_input_rank,
                     info.vocab, info.router_depth, info.input_rank if info.factored else 0)
    hist = np.bincount(lv[:, :, -1].reshape(-1), minlength=info.n_experts)
    log(f"leaves of the last layer: {np.count_nonzero(hist)} of {info.n_experts} used, max share "
        f"{hist.max() / hist.sum():.4f}; compulsory {alg['per_token_compulsory']:.0f} B/token, per-stream "
        f"{alg['per_token_per_stream']:.0f} B/token")

    # timed region: the zero fill of the state is part of each step (one 2 MB fill kernel)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(a.steps):
        launch()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    tokens_per_s = B * T / (ms / 1e3)
    achieved = alg["compulsory"] / (ms / 1e3) / 1e9
    log(f"{a.steps} steps: {ms:.3f} ms/step, {tokens_per_s / 1e6:.2f} M tokens/s, compulsory {achieved:.0f} GB/s "
        f"({achieved / PEAK_HBM_GBS:.3f} of 8 TB/s), per-stream {alg['per_stream'] / (ms / 1e3) / 1e9:.0f} GB/s")

    kernel = (f"ygg::fast_kernel<{info.d_state}, {info.n_layers}>" if info.kernel == 1 else
              f"ygg::run_kernel<{info.d_state}, {info.block_size}, {info.readout_rank}>")
    # HBM bytes per launch measured by rocprofv3 (FETCH_SIZE, WRITE_SIZE, copy-calibrated) for this workload and kernel
    traffic = None
    tf = ROOT / "profiles" / f"traffic_{w.name}.json"
    if tf.exists() and B == w.streams and T == w.steps:
        try:
            doc = json.loads(tf.read_text())
            if doc.get("kernel") == kernel:
                traffic = doc.get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    batch1 = None
    if a.batch1_tokens > 0:
        batch1 = run_batch1(model, w, a.batch1_tokens, L, _lib)
        log(f"batch-1: {batch1}")

    del logits
    torch.cuda.empty_cache()
    cpu = None
    if not a.no_cpu:
        t0 = time.time()
        cpu = cpu_baseline(path, x_np, min(a.cpu_procs, os.cpu_count() or 1), a.cpu_streams)
        log(f"cpu baseline ({time.time() - t0:.1f}s): {cpu}")

    out = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": f"{w.name}: {B} streams x {T} tokens ({w.tokens}, seed {w.token_seed}), model "
                               f"V={info.vocab} L={info.n_layers} n={info.d_state} b={info.block_size} "
                               f"D={info.router_depth} R={info.readout_rank} R2={info.layer_input_rank} "
                               f"(seed {w.model_seed}, {info.file_array_bytes / 1e9:.2f} GB YGG1)",
                   "streams": B, "tokens_per_stream": T, "model_file_bytes": int(info.file_array_bytes),
                   "step": "one ygg_run launch: every token of every stream, logits written per token",
                   "parallelism": "1 GPU (streams independent)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": alg["compulsory"],
                     "compulsory_bytes_per_token": round(alg["per_token_compulsory"], 1),
                     "per_stream_bytes_per_token": round(alg["per_token_per_stream"], 1),
                     "per_stream_GBps": round(alg["per_stream"] / (ms / 1e3) / 1e9, 1),
                     "kernel": kernel},
        "cpu_baseline": cpu,
        "batch1": batch1,
    }
    print(json.dumps(out), flush=True)
    model.close()


def run_batch1(model, w, n_tok: int, L, _lib) -> dict:
    """One stream: (a) one persistent ygg_run launch over n_tok tokens; (b) the per-token ygg_step loop captured in
    hipGraphs of 512 steps each (state in place), replayed back to back. Both write the logits of every token."""
    import torch
    dev = model.device
    x1 = torch.as_tensor(w.make_tokens(1, n_tok)[0], device=dev).contiguous()
    V = model.vocab
    lg = torch.empty(n_tok, V, dtype=torch.float32, device=dev)
    st = model.init_state(1)
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    ptr = lambda t, off=0: ctypes.c_void_p(t.data_ptr() + off)  # noqa: E731
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # (a) persistent launch
    _lib.check(L.ygg_run(model._h, ptr(x1), 1, n_tok, ptr(st), ptr(lg), None, None, None, sp))
    torch.cuda.synchronize()
    st.zero_()
    e0.record(stream)
    _lib.check(L.ygg_run(model._h, ptr(x1), 1, n_tok, ptr(st), ptr(lg), None, None, None, sp))
    e1.record(stream)
    torch.cuda.synchronize()
    run_us = e0.elapsed_time(e1) * 1e3 / n_tok
    ref_logits = lg.clone()
    # (b) graphs of per-token steps
    G = 512
    graphs = []
    st.zero_()
    torch.cuda.synchronize()
    for g0 in range(0, n_tok, G):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for t in range(g0, min(n_tok, g0 + G)):
                _lib.check(L.ygg_step(model._h, ptr(x1, 4 * t), ptr(st), ptr(st), ptr(lg, 4 * t * V), None, 1, cs))
        graphs.append(g)
    st.zero_()
    torch.cuda.synchronize()
    e0.record(stream)
    for g in graphs:
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    graph_us = e0.elapsed_time(e1) * 1e3 / n_tok
    same = bool(torch.equal(lg, ref_logits))
    return {"tokens": n_tok, "us_per_token_persistent_launch": round(run_us, 3),
            "us_per_token_graph_step": round(graph_us, 3), "graph_steps_per_graph": G,
            "graph_logits_equal_persistent": same}


if __name__ == "__main__":
    main()
