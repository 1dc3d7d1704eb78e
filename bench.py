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


# The reference's trained model shapes (configs/{enwik8,hg38}/{small,medium,large}.yaml: 5 layers, block 16, router
# depth 10; state width, readout rank, layer-input rank), as synthetic byte models
REFERENCE_SHAPES = {"small": (64, 8, 16), "medium": (128, 16, 32), "large": (256, 32, 64)}


def workload(cfg: int, storage: str = "table", shape: str = "", scales: str = "tensor"):
    """The configuration's workload; storage "factored" stores its routed inputs factored at rank 64 (the format's
    other storage, cpu/ygg.cpp:339-358: about 0.78 GB for configuration 4 instead of 3.63 GB); shape (one of
    REFERENCE_SHAPES) replaces the configuration's model by a random one of that trained shape (V = 256, Gaussian
    router, seed 5) and keeps its tokens and stream count; scales "group" gives the model group scales (per-group
    state scales, per-row readout scales, per-class unembedding scales: the export's other scale mode,
    cpu/export.py:216-262)."""
    import dataclasses
    from yggdrasil_amd import synth
    w = synth.CONFIGS[cfg]
    if shape:
        n, R, R2 = REFERENCE_SHAPES[shape]
        w = dataclasses.replace(w, name=f"ref_{shape}_d{n}_L5_D10", model_seed=5,
                                spec=synth.ModelSpec(n, 16, 10, 256, 5, R, R2, router="gauss"))
    if storage == "factored":
        w = dataclasses.replace(w, name=w.name + "_factored", spec=dataclasses.replace(w.spec, input_rank=64))
    if scales == "group":
        w = dataclasses.replace(w, name=w.name + "_group", spec=dataclasses.replace(w.spec, group=True))
    return w


def model_path(cfg: int, cache: Path, storage: str = "table", shape: str = "", scales: str = "tensor") -> Path:
    from yggdrasil_amd import synth
    w = workload(cfg, storage, shape, scales)
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


def host_facts() -> dict:
    """The host the CPU baseline runs on: its CPU model, logical CPUs, the CPUs this process may use, and whether
    transparent huge pages are on (the reference allocates its model in huge pages, cpu/ygg.cpp:118-129)."""
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        thp = Path("/sys/kernel/mm/transparent_hugepage/enabled").read_text().strip()
    except OSError:
        thp = ""
    return {"cpu_model": model, "host_logical_cpus": os.cpu_count(),
            "usable_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count(),
            "thp": thp}


# Why the baseline uses at most 16 cores: a one-GPU job on the GPU boxes gets a 16-core share of the host, whatever
# the host's core count; more pinned processes would share cores with the GPU job's own threads.
CPU_SHARE = 16
# The reference binary's target: it is built from cpu/ygg.cpp in the build container (its source does not travel),
# so for any AVX-512 VNNI host rather than the build host's -march=native.
REF_MARCH = "-march=x86-64-v4 -mavx512vnni"
SOFTMAX_NOTE = ("the reference's time mode computes an f32 softmax of every token's logits (cpu/ygg.cpp:61-72, "
                "552), included in its ns/token; the GPU value writes the logits and computes no softmax; the same "
                "softmax on the GPU (ygg_softmax) is timed apart in the line's softmax object")


def cpu_baseline(path: Path, tokens: np.ndarray, procs: int, streams_per_proc: int) -> dict:
    """The reference kernel's `time` mode (cpu/ygg.cpp:528-562) on the host: `procs` processes, each pinned to one
    core, each on its own streams_per_proc streams concatenated into one token stream (state carried, f32 softmax
    per token included, as the reference times itself). Falls back to the C oracle (16 threads) when the reference
    binary is absent or the host lacks AVX-512 VNNI."""
    from oracle import oracle as O
    B, T = tokens.shape
    procs = max(1, min(procs, B))
    streams_per_proc = max(1, min(streams_per_proc, B // procs))
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
                    "sample": f"{procs} pinned processes of `ygg time` (cpu/ygg.cpp, -O3 {REF_MARCH}), each "
                              f"{streams_per_proc} streams of the workload concatenated into {ntok} tokens (first "
                              f"1000 untimed, state carried, f32 softmax per token included); value = sum over "
                              f"processes of 1e9 / mean ns/token",
                    "per_core_median_ns_per_token": round(float(np.median(med)), 1),
                    "per_core_tokens_per_s": round(1e9 / float(np.median(med)), 1),
                    "thp_kB_proc0": int(thp), "wall_s": round(wall, 1), "march": REF_MARCH,
                    "cores_why": f"one pinned process per core of the {CPU_SHARE}-core share a one-GPU job gets on "
                                 f"the GPU box", "softmax": SOFTMAX_NOTE, **host_facts()}
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
                      f"logits only, no softmax", **host_facts()}


def _counter_sums(d: str) -> dict:
    """rocprofv3 --pmc CSV output under d -> {(dispatch id, kernel name): counter value summed over its rows}."""
    import csv
    files = sorted(Path(d).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    out = {}
    for f in files:
        for r in csv.DictReader(open(f)):
            name = r["Kernel_Name"].split("(")[0].strip()
            k = (int(r["Dispatch_Id"]), name[5:] if name.startswith("void ") else name)
            out[k] = out.get(k, 0.0) + float(r["Counter_Value"])
    return out


def traffic_summary(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir, copy_bytes, workload, algorithmic,
                    rdreq_dir=None, kernel=None):
    """HBM bytes of the last step-kernel dispatch from two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE; KiB per
    dispatch), each scaled by bytes moved / counter reading of a plain device copy of copy_bytes. rdreq_dir: a third
    run of TCC_EA0_RDREQ_sum and TCC_EA0_RDREQ_DRAM_sum (128-byte read requests leaving L2, and those addressed to
    the memory controller, behind which the MALL sits)."""
    f, w = _counter_sums(fetch_dir), _counter_sums(write_dir)
    cf, cw = _counter_sums(copy_fetch_dir), _counter_sums(copy_write_dir)
    copies_f = [v for (_, n), v in cf.items() if "copyBuffer" in n]
    copies_w = [v for (_, n), v in cw.items() if "copyBuffer" in n]
    if not copies_f or not copies_w:
        raise SystemExit("no copyBuffer dispatch in the calibration runs")
    ff = copy_bytes / (1024 * float(np.mean(copies_f)))
    wf = copy_bytes / (1024 * float(np.mean(copies_w)))
    pick = (lambda n: n == kernel) if kernel else (lambda n: n.startswith("ygg::"))
    kf = max(k for k in f if pick(k[1]))
    kw = max(k for k in w if pick(k[1]))
    assert kf[1] == kw[1], (kf, kw)
    fetched, written = f[kf] * 1024 * ff, w[kw] * 1024 * wf
    doc = {"workload": workload, "kernel": kf[1], "fetch_size_kib": f[kf], "write_size_kib": w[kw],
           "copy_calibration": {"bytes": copy_bytes, "fetch_size_kib": float(np.mean(copies_f)),
                                "write_size_kib": float(np.mean(copies_w)), "fetch_factor": round(ff, 4),
                                "write_factor": round(wf, 4)},
           "hbm_bytes_per_launch": int(fetched + written), "fetched_bytes": int(fetched),
           "written_bytes": int(written)}
    if algorithmic:
        doc["algorithmic_bytes_per_launch"] = int(algorithmic)
        doc["traffic_over_algorithmic"] = round((fetched + written) / algorithmic, 3)
    if rdreq_dir:
        import csv
        by = {}
        for fcsv in sorted(Path(rdreq_dir).rglob("*counter_collection.csv")):
            for r in csv.DictReader(open(fcsv)):
                name = r["Kernel_Name"].split("(")[0].strip()
                name = name[5:] if name.startswith("void ") else name
                if name == kf[1]:
                    k = (int(r["Dispatch_Id"]), r["Counter_Name"])
                    by[k] = by.get(k, 0.0) + float(r["Counter_Value"])
        last = max(d for d, _ in by)
        rq, dr = by.get((last, "TCC_EA0_RDREQ_sum"), 0.0), by.get((last, "TCC_EA0_RDREQ_DRAM_sum"), 0.0)
        doc["read_requests_128B"] = int(rq)
        doc["read_requests_to_memory_controller_128B"] = int(dr)
        doc["mall_split"] = ("none measurable: every L2 read request is addressed to the memory controller, which "
                             "serves MALL hits and HBM reads alike; traffic counts both") if rq and dr == rq else \
            f"{dr / rq:.4f} of the read requests go to the memory controller" if rq else None
    return doc


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--traffic":
        # python bench.py --traffic FETCH_DIR WRITE_DIR COPY_FETCH_DIR COPY_WRITE_DIR COPY_BYTES BENCH_JSON OUT_JSON
        #                           [RDREQ_DIR]
        fd, wd, cfd, cwd, cb, bj, out = sys.argv[2:9]
        rdq = sys.argv[9] if len(sys.argv) > 9 else None
        b = json.loads(Path(bj).read_text().strip().splitlines()[-1])
        wl = b["config"]["workload"].split(" (")[0]
        doc = traffic_summary(fd, wd, cfd, cwd, int(cb), wl, b["roofline"]["algorithmic_bytes_per_launch"], rdq,
                              b["roofline"]["kernel"])
        Path(out).write_text(json.dumps(doc, indent=1) + "\n")
        print(json.dumps(doc))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=4, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--storage", default="table", choices=["table", "factored"],
                    help="routed-layer input storage of the synthetic model (factored: rank 64)")
    ap.add_argument("--shape", default="", choices=["", *REFERENCE_SHAPES],
                    help="a model of one of the reference's trained shapes instead of the configuration's")
    ap.add_argument("--scales", default="tensor", choices=["tensor", "group"],
                    help="state/readout/unembedding scales of the synthetic model")
    ap.add_argument("--streams", type=int, default=0, help="override the configuration's stream count")
    ap.add_argument("--tokens", type=int, default=0, help="override the configuration's tokens per stream")
    ap.add_argument("--cache", default=os.environ.get("YGG_BENCH_DIR", os.path.join(tempfile.gettempdir(),
                                                                                      "ygg_bench")))
    ap.add_argument("--batch1-tokens", type=int, default=8192)
    ap.add_argument("--cpu-procs", type=int, default=CPU_SHARE)
    ap.add_argument("--cpu-streams", type=int, default=256, help="streams per CPU baseline process")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-float", action="store_true", help="skip the float step's batch-1 leg")
    ap.add_argument("--entry", default="run", choices=["run", "grouped"],
                    help="the timed C-ABI call: ygg_run (per-stream kernels) or ygg_run_grouped (leaf-grouped "
                         "phases, MFMA tiles from YGG_GROUP_MFMA_MIN streams)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py runs on one GPU only: the streams are independent, so N GPUs would each run this same "
              f"workload on their own share with no communication (requested --gpus {a.gpus}).", file=sys.stderr)
        sys.exit(2)

    import torch
    from yggdrasil_amd import synth
    from yggdrasil_amd.inference import Yggdrasil
    from yggdrasil_amd.roofline import step_bytes

    w = workload(a.config, a.storage, a.shape, a.scales)
    B, T = a.streams or w.streams, a.tokens or w.steps
    path = model_path(a.config, Path(a.cache), a.storage, a.shape, a.scales)
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

    entry = L.ygg_run_grouped if a.entry == "grouped" else L.ygg_run
    if a.entry == "grouped" and not info.grouped:
        raise SystemExit("ygg_run_grouped does not take this model")

    def launch(with_leaves=False):
        st.zero_()
        _lib.check(entry(model._h, p(x), B, T, p(st), p(logits), p(leaves) if with_leaves else None, None,
                         None, sp))

    # the first warmup launch also records the leaves, for the compulsory-byte count
    for i in range(max(1, a.warmup)):
        launch(with_leaves=(i == 0))
    torch.cuda.synchronize()
    lv = leaves.cpu().numpy()
    del leaves
    alg = step_bytes(lv, x_np, info.d_state, info.block_size, info.readout_rank, info.layer_input_rank,
                     info.vocab, info.router_depth, info.input_rank if info.factored else 0, group=bool(info.group))
    hist = np.bincount(lv[:, :, -1].reshape(-1), minlength=info.n_experts)
    log(f"leaves of the last layer: {np.count_nonzero(hist)} of {info.n_experts} used, max share "
        f"{hist.max() / hist.sum():.4f}; compulsory {alg['per_token_compulsory']:.0f} B/token, per-stream "
        f"{alg['per_token_per_stream']:.0f} B/token")

    # timed region: the zero fill of the state is part of each step (one 2 MB fill kernel); a second pair of events
    # on the same stream brackets each step kernel alone, for its average duration
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    e0, e1 = ev(), ev()
    ks = [(ev(), ev()) for _ in range(a.steps)]
    torch.cuda.synchronize()
    e0.record(stream)
    for k0, k1 in ks:
        st.zero_()
        k0.record(stream)
        _lib.check(entry(model._h, p(x), B, T, p(st), p(logits), None, None, None, sp))
        k1.record(stream)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    kernel_ms = sum(k0.elapsed_time(k1) for k0, k1 in ks) / a.steps
    tokens_per_s = B * T / (ms / 1e3)
    achieved = alg["compulsory"] / (kernel_ms / 1e3) / 1e9
    log(f"{a.steps} steps: {ms:.3f} ms/step ({kernel_ms:.3f} ms in the step kernel), {tokens_per_s / 1e6:.2f} M "
        f"tokens/s, compulsory {achieved:.0f} GB/s ({achieved / PEAK_HBM_GBS:.3f} of 8 TB/s), per-stream "
        f"{alg['per_stream'] / (kernel_ms / 1e3) / 1e9:.0f} GB/s")

    grouped_graph = None
    if a.entry == "grouped":
        # the same call captured in one hipGraph (its 3 L T launches as nodes; the workspace already sized) and
        # replayed: what capture saves over launching each phase from the host
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            _lib.check(entry(model._h, p(x), B, T, p(st), p(logits), None, None, None, cs))
        st.zero_()
        g.replay()
        torch.cuda.synchronize()
        g0, g1 = ev(), ev()
        st.zero_()
        g0.record(stream)
        g.replay()
        g1.record(stream)
        torch.cuda.synchronize()
        grouped_graph = {"ms": round(g0.elapsed_time(g1), 4), "launches": 3 * info.n_layers * T + 1}
        log(f"grouped call replayed from one hipGraph: {grouped_graph}")
        del g

    kernel = model.kernel_name(B, T) if a.entry == "run" else \
        f"ygg_run_grouped: grp_route, grp_plan, grp_update per (token, layer), MFMA tiles from " \
        f"{os.environ.get('YGG_GROUP_MFMA_MIN', '8')} streams"
    # HBM bytes per launch measured by rocprofv3 (FETCH_SIZE, WRITE_SIZE, copy-calibrated) for this workload and kernel
    traffic, traffic_detail = None, None
    tf = ROOT / "profiles" / f"traffic_{w.name}.json"
    if tf.exists() and B == w.streams and T == w.steps:
        try:
            doc = json.loads(tf.read_text())
            if doc.get("kernel") == kernel:
                traffic = doc.get("hbm_bytes_per_launch")
                traffic_detail = {k: doc[k] for k in ("fetched_bytes", "written_bytes", "traffic_over_algorithmic",
                                                      "read_requests_128B", "read_requests_to_memory_controller_128B",
                                                      "mall_split") if k in doc}
                traffic_detail["source"] = f"profiles/{tf.name}"
        except (OSError, ValueError):
            traffic, traffic_detail = None, None

    # the f32 softmax of every logit row (what the reference's time mode adds per token), timed apart from the step
    sm = None
    if a.entry == "run":
        pr = torch.empty_like(logits)
        s0, s1 = ev(), ev()
        _lib.check(L.ygg_softmax(p(logits), B * T, info.vocab, p(pr), None, sp))
        s0.record(stream)
        _lib.check(L.ygg_softmax(p(logits), B * T, info.vocab, p(pr), None, sp))
        s1.record(stream)
        torch.cuda.synchronize()
        sm_ms = s0.elapsed_time(s1)
        sm = {"ms": round(sm_ms, 4), "rows": B * T,
              "GBps": round(2 * 4 * B * T * info.vocab / (sm_ms / 1e3) / 1e9, 1),
              "step_plus_softmax_tokens_per_s": round(B * T / ((kernel_ms + sm_ms) / 1e3), 1)}
        log(f"softmax of {B * T} rows: {sm}")
        del pr

    # the score mode on the same streams (ygg_score: the step and the float64 NLL of each token's next token, the
    # last token of a stream scored against its first; no logits written), timed like the step
    score = None
    if a.entry == "run":
        yt = torch.roll(x, -1, dims=1).contiguous()
        nll = torch.zeros(B, dtype=torch.float64, device=dev)

        def score_launch():
            st.zero_()
            _lib.check(L.ygg_score(model._h, p(x), p(yt), B, T, p(st), p(nll), sp))
        score_launch()
        torch.cuda.synchronize()
        c0, c1 = ev(), ev()
        c0.record(stream)
        for _ in range(a.steps):
            score_launch()
        c1.record(stream)
        torch.cuda.synchronize()
        sc_ms = c0.elapsed_time(c1) / a.steps
        score = {"ms": round(sc_ms, 4), "tokens_per_s": round(B * T / (sc_ms / 1e3), 1),
                 "over_run_step": round(sc_ms / ms, 4), "kernel": model.kernel_name(B, T, score=True)}
        log(f"score: {score}")
        del yt, nll

    batch1 = None
    if a.batch1_tokens > 0 and a.entry == "run":
        batch1 = run_batch1(model, w, a.batch1_tokens, L, _lib)
        log(f"batch-1: {batch1}")

    del logits
    torch.cuda.empty_cache()
    float_b1 = None
    if not a.no_float and a.entry == "run":
        float_b1 = run_float_batch1()
        log(f"float batch-1: {float_b1}")
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
                   "step": f"one {'ygg_run launch' if a.entry == 'run' else 'ygg_run_grouped call'}: every token "
                           f"of every stream, logits written per token",
                   "parallelism": "1 GPU (streams independent)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic, "traffic_detail": traffic_detail,
                     "algorithmic_bytes_per_launch": alg["compulsory"],
                     "compulsory_bytes_per_token": round(alg["per_token_compulsory"], 1),
                     "per_stream_bytes_per_token": round(alg["per_token_per_stream"], 1),
                     "per_stream_GBps": round(alg["per_stream"] / (kernel_ms / 1e3) / 1e9, 1),
                     "kernel": kernel, "kernel_ms": round(kernel_ms, 4)},
        "cpu_baseline": cpu,
        "softmax": sm,
        "score": score,
        "grouped_graph": grouped_graph,
        "batch1": batch1,
        "float_batch1": float_b1,
    }
    print(json.dumps(out), flush=True)
    model.close()


def run_batch1(model, w, n_tok: int, L, _lib) -> dict:
    """One stream of n_tok known tokens: (a) one persistent ygg_run launch; (a') the same followed by ygg_softmax over
    its rows (the reference's time mode: known tokens, state carried, an f32 softmax per token), eagerly and captured
    in one hipGraph; (b) the per-token ygg_step loop captured in hipGraphs of 512 steps each (state in place, a launch
    per token, as a caller whose every token depends on the last would run); (c) greedy generation on the device."""
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
    # the reference's time mode also takes the f32 softmax of every token's logits (cpu/ygg.cpp:545-553): the same
    # persistent launch followed by ygg_softmax over its n_tok rows
    pr = torch.empty_like(lg)
    ls = torch.empty(n_tok, dtype=torch.float32, device=dev)
    st.zero_()
    torch.cuda.synchronize()
    e0.record(stream)
    _lib.check(L.ygg_run(model._h, ptr(x1), 1, n_tok, ptr(st), ptr(lg), None, None, None, sp))
    _lib.check(L.ygg_softmax(ptr(lg), n_tok, V, ptr(pr), ptr(ls), sp))
    e1.record(stream)
    torch.cuda.synchronize()
    time_mode_us = e0.elapsed_time(e1) * 1e3 / n_tok
    # the same run captured in one hipGraph (the launch and the softmax as its two nodes) and replayed: the batch-1
    # latency run of the whole token file, as `ygg time` runs it on the host
    g1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(L.ygg_run(model._h, ptr(x1), 1, n_tok, ptr(st), ptr(lg), None, None, None, cs))
        _lib.check(L.ygg_softmax(ptr(lg), n_tok, V, ptr(pr), ptr(ls), cs))
    st.zero_()
    g1.replay()
    st.zero_()
    torch.cuda.synchronize()
    e0.record(stream)
    g1.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    graph_run_us = e0.elapsed_time(e1) * 1e3 / n_tok
    graph_run_same = bool(torch.equal(lg, ref_logits))
    del g1, pr, ls
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
    # (c) greedy generation on the device: one ygg_generate launch samples n_tok tokens, each fed back as the next
    # input, so no two layers of different tokens overlap (each token waits for the last layer of the one before)
    out = torch.empty(1, n_tok, dtype=torch.int32, device=dev)
    st.zero_()
    _lib.check(L.ygg_generate(model._h, ptr(x1), 1, 64, ptr(st), ctypes.c_float(0.0), 0, ctypes.c_uint64(0),
                              ptr(out), None, sp))
    st.zero_()
    torch.cuda.synchronize()
    model.spec_stats(reset=True)
    e0.record(stream)
    _lib.check(L.ygg_generate(model._h, ptr(x1), 1, n_tok, ptr(st), ctypes.c_float(0.0), 0, ctypes.c_uint64(0),
                              ptr(out), None, sp))
    e1.record(stream)
    torch.cuda.synchronize()
    gen_us = e0.elapsed_time(e1) * 1e3 / n_tok
    # the generation's steps taken from the speculating helpers' slots (all zero without that build)
    spec = model.spec_stats()
    return {"tokens": n_tok, "us_per_token_persistent_launch": round(run_us, 3),
            "us_per_token_time_mode": round(time_mode_us, 3),
            "us_per_token_graph_run": round(graph_run_us, 3), "graph_run_logits_equal_persistent": graph_run_same,
            "us_per_token_graph_step": round(graph_us, 3), "graph_steps_per_graph": G,
            "graph_logits_equal_persistent": same, "us_per_token_generate_greedy": round(gen_us, 3),
            "generate_spec": spec,
            "kernels": {"persistent_launch": model.kernel_name(1, n_tok), "graph_step": model.kernel_name(1, 1),
                        "generate": model.kernel_name(1, n_tok, generate=True)}}


# The reference's float GPU figure: its Triton step (yggdrasil/inference_triton.py:196-212, replayed from a CUDA
# graph) at batch 1 on the large trained model, README.md:43
REF_FLOAT_GPU_US = 80.1


def run_float_batch1(n_tok: int = 1024, graph_steps: int = 256) -> dict:
    """The float step (the f32 float kernel of a .npz checkpoint, FloatYggdrasil) at batch 1, on a random checkpoint of
    the reference's large trained shape (configs/enwik8/large.yaml: 5 layers, d_state 256, block 16, router depth
    10, router token dim 16, input rank 64, readout rank 32, layer-input rank 64; seed 5): (a) one launch of n_tok
    known tokens, state carried; (b) a per-token step loop (one ygg_float_run of one token, state in place) captured
    in a hipGraph of graph_steps steps and replayed, as the reference's Triton backend replays its step."""
    import torch
    from yggdrasil_amd import _lib
    from yggdrasil_amd.float_model import FloatSpec, FloatYggdrasil, float_layers, from_params, random_params
    spec = FloatSpec(d_state=256, block_size=16, router_depth=10, vocab=256, n_layers=5, router_token_dim=16,
                     input_rank=64, readout_rank=32, layer_input_rank=64)
    # the checkpoint's arrays in memory (random_checkpoint's, without the 0.8 GB file), tables by matrix products
    t0 = time.time()
    raw, ob = from_params(random_params(spec, 5))
    fm = FloatYggdrasil(float_layers(raw, blas=True), ob, precision=32)
    del raw
    log(f"float model (large shape) built in {time.time() - t0:.1f}s")
    from yggdrasil_amd import synth
    L = _lib.lib()
    dev = fm.device
    x = torch.as_tensor(synth.zipf_bytes(1, n_tok, 11)[0], dtype=torch.int32, device=dev).contiguous()
    st = fm.init_state(1)
    lg = torch.empty(n_tok, fm.classes, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    ptr = lambda t, off=0: ctypes.c_void_p(t.data_ptr() + off)  # noqa: E731
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _lib.check(L.ygg_float_run(fm._h, ptr(x), 1, n_tok, ptr(st), ptr(lg), None, None, sp))
    st.zero_()
    torch.cuda.synchronize()
    e0.record(stream)
    _lib.check(L.ygg_float_run(fm._h, ptr(x), 1, n_tok, ptr(st), ptr(lg), None, None, sp))
    e1.record(stream)
    torch.cuda.synchronize()
    run_us = e0.elapsed_time(e1) * 1e3 / n_tok
    ref = lg[:graph_steps].clone()
    g = torch.cuda.CUDAGraph()
    st.zero_()
    with torch.cuda.graph(g):
        cs = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for t in range(graph_steps):
            _lib.check(L.ygg_float_run(fm._h, ptr(x, 4 * t), 1, 1, ptr(st), ptr(lg, 4 * t * fm.classes), None, None,
                                       cs))
    st.zero_()
    g.replay()
    torch.cuda.synchronize()
    st.zero_()
    torch.cuda.synchronize()
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    step_us = e0.elapsed_time(e1) * 1e3 / graph_steps
    same = bool(torch.equal(lg[:graph_steps], ref))
    del g
    fm.close()
    return {"model": "random f32 checkpoint of configs/enwik8/large.yaml's shape (5 layers, d_state 256, D 10, R 32, "
                     "R2 64, input rank 64; seed 5)",
            "tokens": n_tok, "us_per_token_run": round(run_us, 3), "us_per_token_graph_step": round(step_us, 3),
            "graph_steps_per_graph": graph_steps, "graph_logits_equal_run": same,
            "reference_triton_us_per_token": REF_FLOAT_GPU_US, "reference_source": "README.md:43 (GPU µs/tok)",
            "kernel": fm.kernel_name}


if __name__ == "__main__":
    main()
