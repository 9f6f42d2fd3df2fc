#!/usr/bin/env python3
"""IQ2_XXS matmul throughput on one MI355X (gfx950).

Metric: "IQ2_XXS matmul GB/s (%HBM peak) at M=1; TFLOP/s (%MFMA
peak) at M=512".

Workload of the headline line: one decode step of a
Llama-3-8B MLP at M=1 with IQ2_XXS weights — gate (K=4096, N=14336), up (same
shape) and down (K=14336, N=4096) — three launches of the GEMV kernel on one
stream.  Synthetic seeded weights (d = f16(|N(0,1)|*1e-3), uniform codes) and
N(0,1) fp32 activations; no checkpoints.

  value   = algorithmic bytes of the K timed steps / elapsed time (GB/s), with
            inputs resident in HBM.  Algorithmic bytes per matmul:
            N*ceil(K/256)*66 + M*K*4 + M*N*4.
  timing  = HIP events recorded on the launch stream around one replay of a HIP
            graph holding the K steps; every step uses a different copy of the
            weights, and the copies total >= 512 MB so the 256 MB Infinity Cache
            cannot serve them.
  roofline.achieved = per-launch algorithmic bytes / mean launch duration.

The prefill line (M=512, K=4096, N=14336, f16 activations) is
reported in the same JSON object under "prefill_m512" (TFLOP/s, %MFMA f16 peak).
The CPU baseline is the oracle (a C restatement of the reference's scalar CPU
reference) run on the host cores over the same decode step.

`--gpus N` with N > 1 exits: this build targets one GPU.
"""

from __future__ import annotations

import argparse
import importlib.util
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(REPO, "candelora-metal-kernels_amd")

HBM_PEAK_GBS = 8000.0         # MI355X HBM3E, 8 TB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA
MALL_BYTES = 256 << 20

METRIC = "IQ2_XXS matmul GB/s (%HBM peak) at M=1; TFLOP/s (%MFMA peak) at M=512"
TRAFFIC_FILE = os.path.join(REPO, "profiles", "gemv_config1_traffic.json")
# Sources of the one-row GEMV: the traffic file records their digest when its
# counters are summarised, and the bench line reports the traffic figure only
# while the digest still matches (a stale figure is reported as null).
GEMV_SOURCES = ["csrc/iq2xxs_gemv.hip", "csrc/iq2xxs_gemv_common.h", "csrc/iq2xxs_device.h",
                "csrc/iq2xxs_format.h", "csrc/iq2xxs_kernels.h", "csrc/iq_rows_formats.h"]

DECODE_SHAPES = [("gate", 4096, 14336), ("up", 4096, 14336), ("down", 14336, 4096)]
# Untimed decode steps replayed right before the timed replay (about 7 ms of
# work at the current speed), so the timed steps run at steady-state clocks.
DECODE_WARM_STEPS = 300
DECODE_STAT_REPLAYS = 10


def nearest_rank(sorted_values, p):
    """Nearest-rank percentile of sorted values (as the reference's bench)."""
    rank = max(1, math.ceil(p * len(sorted_values)))
    return sorted_values[min(rank, len(sorted_values)) - 1]


def load_package():
    name = "candelora_metal_kernels_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(
        name, os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def alg_bytes(m, k, n, xbytes=4):
    return n * math.ceil(k / 256) * 66 + m * k * xbytes + m * n * 4


def gemv_source_digest():
    """sha256 (first 16 hex digits) over the one-row GEMV's source files."""
    import hashlib
    h = hashlib.sha256()
    for rel in GEMV_SOURCES:
        h.update(rel.encode())
        with open(os.path.join(PKG_DIR, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def _counter_rows(run_dir):
    """(kernel name, counter name, value) per dispatch from a rocprofv3
    `--pmc ... --output-format csv` output folder."""
    import csv
    import glob
    files = sorted(glob.glob(os.path.join(run_dir, "**", "*counter_collection.csv"),
                             recursive=True))
    if not files:
        raise SystemExit(f"bench.py: no *counter_collection.csv under {run_dir}")
    rows = []
    for path in files:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append((r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"]),
                             r.get("Dispatch_Id", "")))
    return rows


def traffic_summary(root, out_path):
    """Summarise the four counter passes under `root` (copy_FETCH_SIZE,
    gemv_FETCH_SIZE, copy_WRITE_SIZE, gemv_WRITE_SIZE) into `out_path`.

    Each counter is calibrated by what it reads for the 256 MiB device copy of
    `--copy-calibration` (read 256 MiB, write 256 MiB); the GEMV figure is the
    mean KiB per dispatch over every one-row GEMV launch of the run."""
    copy_bytes = 256 << 20
    res = {}
    names = set()
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        cal = sorted(v for k, c, v, _ in _counter_rows(os.path.join(root, "copy_" + counter))
                     if c == counter and "copyBuffer" in k)
        if not cal:
            raise SystemExit(f"bench.py: no copyBuffer dispatch in copy_{counter}")
        cal_kib = cal[len(cal) // 2]
        factor = copy_bytes / (cal_kib * 1024.0)
        per_shape = {}
        for k, c, v, _ in _counter_rows(os.path.join(root, "gemv_" + counter)):
            if c == counter and "iq2xxs_gemv_kernel" in k:
                per_shape.setdefault(k, []).append(v)
                names.add(k)
        if not per_shape:
            raise SystemExit(f"bench.py: no one-row GEMV dispatch in gemv_{counter}")
        allv = [v for vs in per_shape.values() for v in vs]
        res[counter] = {"factor": factor, "calibration_kib": cal_kib,
                        "mean_kib": sum(allv) / len(allv), "dispatches": len(allv),
                        "per_kernel_mean_kib": {k: sum(vs) / len(vs)
                                                for k, vs in per_shape.items()}}
    fetch = res["FETCH_SIZE"]["mean_kib"] * 1024 * res["FETCH_SIZE"]["factor"]
    write = res["WRITE_SIZE"]["mean_kib"] * 1024 * res["WRITE_SIZE"]["factor"]
    alg = sum(alg_bytes(1, k, n) for _, k, n in DECODE_SHAPES) / len(DECODE_SHAPES)
    summary = {
        "kernels": sorted(names),
        "workload": "config 1 decode step: gate K=4096 N=14336, up K=4096 N=14336, "
                    "down K=14336 N=4096 (M=1, fp32 x)",
        "source_digest": gemv_source_digest(),
        "hbm_bytes_per_launch": round(fetch + write),
        "fetch_bytes_per_launch": round(fetch),
        "write_bytes_per_launch": round(write),
        "algorithmic_bytes_per_launch": round(alg),
        "fetch_size_factor": round(res["FETCH_SIZE"]["factor"], 4),
        "write_size_factor": round(res["WRITE_SIZE"]["factor"], 4),
        "counters": res,
        "note": "mean over gate/up/down launches of FETCH_SIZE and WRITE_SIZE (KiB per "
                "dispatch) times the factor a 256 MiB device copy needs to read 256 MiB / "
                "write 256 MiB",
    }
    with open(out_path, "w") as f:
        json.dump(summary, f, indent=1)
        f.write("\n")
    print(json.dumps({k: summary[k] for k in ("hbm_bytes_per_launch", "fetch_bytes_per_launch",
                                              "write_bytes_per_launch",
                                              "algorithmic_bytes_per_launch",
                                              "source_digest")}))


def load_traffic():
    """(bytes per launch or None, source note) from the committed traffic file;
    None when the file was measured on other GEMV sources than these."""
    if not os.path.exists(TRAFFIC_FILE):
        return None, "no traffic file"
    try:
        t = json.load(open(TRAFFIC_FILE))
    except (OSError, ValueError) as e:
        return None, f"traffic file unreadable: {e}"
    now = gemv_source_digest()
    if t.get("source_digest") != now:
        return None, (f"profiles/gemv_config1_traffic.json was measured on GEMV sources "
                      f"{t.get('source_digest')}, not these ({now}): not reported")
    return t.get("hbm_bytes_per_launch"), (
        "profiles/gemv_config1_traffic.json: rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, "
        f"copy-calibrated, measured on these GEMV sources ({now}); read from the file, not "
        "measured in this run")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def replay_timed(torch, cabi, graph, sh, steps, warm_steps):
    """Milliseconds of one replay of `graph` (holding `steps` steps) on stream sh.

    The timed replay is preceded, with no host synchronisation in between, by
    untimed replays of the same graph covering at least `warm_steps` steps:
    after a host synchronisation the GPU idles and its clocks take a few
    milliseconds to ramp back up, so a short replay timed straight after one
    would measure the ramp instead of the sustained rate."""
    pre = max(1, math.ceil(warm_steps / max(1, steps)))
    start, stop = cabi.Event(), cabi.Event()
    for _ in range(pre):
        graph.replay()
    start.record(sh)
    graph.replay()
    stop.record(sh)
    torch.cuda.synchronize()
    return start.elapsed_ms(stop)


class Matmul:
    """One preallocated launch through the C ABI (no Python-side allocation).

    Holds references to its tensors: the launch only carries raw device
    pointers, so the tensors must stay alive as long as the launch (or a graph
    that captured it) can run."""

    def __init__(self, cabi, x, wb, ws, out, m, k, n, x_dtype, stream, variant=0, mode=0):
        # the workspace the path asks for (f32 rows staged for the GEMM), allocated once here
        import torch
        ws_bytes = cabi.workspace_size(x_dtype, m, n, k, variant, mode)
        self.workspace = (torch.empty((ws_bytes,), dtype=torch.uint8, device=x.device)
                          if ws_bytes else None)
        self.tensors = (x, wb, ws, out)
        self.args = (x.data_ptr(), x_dtype, x.numel(), m, wb.data_ptr(), wb.numel(),
                     ws.data_ptr(), ws.numel(), n, k, out.data_ptr())
        self.ws_args = ((self.workspace.data_ptr(), ws_bytes) if ws_bytes else (None, 0))
        self.cabi = cabi
        self.stream = stream
        self.variant = variant
        self.mode = mode

    def __call__(self):
        self.cabi.matmul_raw(*self.args, variant=self.variant, mode=self.mode,
                             workspace_ptr=self.ws_args[0], workspace_bytes=self.ws_args[1],
                             stream=self.stream)


def bench_decode(pkg, torch, stream, steps, warmup):
    """All launches, the graph capture and the events use `stream` (a non-default
    stream): work captured into a graph must be issued on the capturing stream."""
    cabi, inputs = pkg.cabi, pkg.inputs
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    step_w_bytes = sum(n * math.ceil(k / 256) * 66 for _, k, n in DECODE_SHAPES)
    copies = max(2, math.ceil(2 * MALL_BYTES / step_w_bytes))
    log(f"[bench] decode: {copies} weight copies x {step_w_bytes/1e6:.2f} MB per step")
    mats = []
    for name, k, n in DECODE_SHAPES:
        wb, ws = inputs.synthetic_weights(n, k)
        wbt = torch.from_numpy(wb).to(dev)
        wst = torch.from_numpy(ws).to(dev)
        reps = [(wbt, wst)] + [(wbt.clone(), wst.clone()) for _ in range(copies - 1)]
        x = torch.from_numpy(inputs.synthetic_x(1, k)).to(dev)
        out = torch.empty((1, n), dtype=torch.float32, device=dev)
        calls = [Matmul(cabi, x, r[0], r[1], out, 1, k, n, cabi.CMK_F32, sh) for r in reps]
        mats.append((name, k, n, calls, out))
    torch.cuda.synchronize()

    def run(i):
        c = i % copies
        for _, _, _, calls, _ in mats:
            calls[c]()

    log(f"[bench] decode: eager warm-up, {max(warmup, copies)} steps on stream {sh:#x}")
    for i in range(max(warmup, copies)):  # eager warm-up (also sets kernel attributes)
        run(i)
    torch.cuda.synchronize()

    log(f"[bench] decode: capturing {steps} steps into a HIP graph")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            run(i)
    log("[bench] decode: untimed replay")
    graph.replay()  # untimed replay (replays on the current stream)
    torch.cuda.synchronize()

    # graph replays must reproduce the eager result of the same launches
    eager = []
    for _, _, _, calls, out in mats:
        calls[(steps - 1) % copies]()
        eager.append(out.clone())
    graph.replay()
    torch.cuda.synchronize()
    for (name, _, _, _, out), e in zip(mats, eager):
        if not torch.equal(out, e):
            raise RuntimeError(f"graph replay differs from eager launch for {name}")

    torch.cuda.synchronize()
    ms = replay_timed(torch, cabi, graph, sh, steps, DECODE_WARM_STEPS)
    step_bytes = sum(alg_bytes(1, k, n) for _, k, n in DECODE_SHAPES)
    launches = steps * len(DECODE_SHAPES)
    # the spread over further timed replays of the same graph (each after an
    # untimed one): median and p95 of their mean launch times
    per_replay = sorted(replay_timed(torch, cabi, graph, sh, steps, 1) * 1e3 / launches
                        for _ in range(DECODE_STAT_REPLAYS))
    return {
        "ms": ms,
        "step_bytes": step_bytes,
        "launches": launches,
        "mean_launch_us": ms * 1e3 / launches,
        "per_launch_bytes": step_bytes / len(DECODE_SHAPES),
        "launch_us_over_replays": {"replays": DECODE_STAT_REPLAYS,
                                   "median": nearest_rank(per_replay, 0.50),
                                   "p95": nearest_rank(per_replay, 0.95),
                                   "min": per_replay[0], "max": per_replay[-1]},
    }


def bench_reference_workload(pkg, torch, stream, warmup=5, runs=20, m=1, n=4096, k=4096):
    """The reference bench's default workload and timing, for continuity with
    it (examples/iq2_matmul_bench.rs:103-118 defaults, 251-324 per format):
    every format at M=1, N=K=4096, f16 x, its LCG inputs (seeds xor'ed with
    the dims, every d = 1.0), one weight set (resident in the caches, as
    there).  Each run is one launch followed by a device synchronize, after
    `warmup` such runs; it is timed twice: on the host around launch +
    synchronize, as the reference times it, and by HIP events on the launch
    stream (the kernel alone).  mean / p50 / p95 (nearest rank) in ms and
    matmuls per second from the host mean, the reference's columns."""
    cabi, inputs = pkg.cabi, pkg.inputs
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    res = {}
    for v, name in enumerate(("iq2-xxs", "iq2-xs", "iq2-s", "iq3-s")):
        x, wb, ws = inputs.reference_bench_case_variant(v, m, n, k)
        xt = torch.from_numpy(x).to(dev).to(torch.float16)
        wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
        out = torch.empty((m, n), dtype=torch.float32, device=dev)
        call = Matmul(cabi, xt, wbt, wst, out, m, k, n, cabi.CMK_F16, sh, variant=v)
        start, stop = cabi.Event(), cabi.Event()
        for _ in range(warmup):
            call()
            torch.cuda.synchronize()
        host, device = [], []
        for _ in range(runs):
            t0 = time.perf_counter()
            start.record(sh)
            call()
            stop.record(sh)
            torch.cuda.synchronize()
            host.append((time.perf_counter() - t0) * 1e3)
            device.append(start.elapsed_ms(stop))
        row = {}
        for label, times in (("host", host), ("device", device)):
            mean = sum(times) / len(times)
            times.sort()
            row[label] = {"mean_ms": mean, "p50_ms": nearest_rank(times, 0.50),
                          "p95_ms": nearest_rank(times, 0.95)}
        hm = row["host"]["mean_ms"]
        row["matmuls_per_s"] = 1e3 / hm if hm > 0 else 0.0
        res[name] = row
        log(f"[bench] reference workload {name}: host mean {hm * 1e3:.1f} us "
            f"(p95 {row['host']['p95_ms'] * 1e3:.1f}), kernel mean "
            f"{row['device']['mean_ms'] * 1e3:.2f} us (p95 {row['device']['p95_ms'] * 1e3:.2f})")
    res["workload"] = (f"examples/iq2_matmul_bench.rs defaults: m={m}, out_dim={n}, in_dim={k}, "
                       f"f16 x, LCG inputs (d = 1), warmup {warmup}, runs {runs}")
    return res


def bench_read_floor(pkg, torch, stream, steps):
    """The plain-read floor beside the decode line: libcmk_probe.so's kernel
    reading the bytes of one decode launch (the mean of the three launches'
    algorithmic bytes, 16-byte loads, no decoding) from rotated buffers, timed
    like the decode line (one graph of `steps` launches, events around a
    replay that follows untimed ones)."""
    import ctypes
    cabi = pkg.cabi
    path = os.path.join(os.path.dirname(cabi.LIB_PATH), "libcmk_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build with __graft_entry__.build()")
    probe = ctypes.CDLL(path)
    probe.cmk_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_void_p]
    probe.cmk_probe_read.restype = ctypes.c_int
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    nbytes = sum(alg_bytes(1, k, n) for _, k, n in DECODE_SHAPES) // len(DECODE_SHAPES)
    nbytes = (nbytes + 15) // 16 * 16
    copies = max(2, math.ceil(2 * MALL_BYTES / nbytes))
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=dev) for _ in range(copies)]
    blocks = 4096
    sink = torch.zeros(blocks, dtype=torch.int32, device=dev)

    def run(i):
        rc = probe.cmk_probe_read(bufs[i % copies].data_ptr(), nbytes, sink.data_ptr(), blocks,
                                  sh)
        if rc != 0:
            raise RuntimeError(f"cmk_probe_read failed: hip error {rc}")

    for i in range(copies):
        run(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            run(i)
    graph.replay()
    torch.cuda.synchronize()
    us = replay_timed(torch, cabi, graph, sh, steps, DECODE_WARM_STEPS) * 1e3 / steps
    log(f"[bench] read floor: {nbytes/1e6:.2f} MB in {us:.2f} us per launch "
        f"({nbytes / (us * 1e-6) / 1e9:.1f} GB/s)")
    return {"bytes": nbytes, "us_per_launch": us, "gbs": nbytes / (us * 1e-6) / 1e9,
            "kernel": "probe_read_kernel (libcmk_probe.so; 4096 x 256 threads, 16-byte "
                      "nontemporal loads)", "launches": steps}


def bench_prefill(pkg, torch, stream, steps, warmup, m=512, k=4096, n=14336):
    cabi, inputs = pkg.cabi, pkg.inputs
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    wb, ws = inputs.synthetic_weights(n, k)
    wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
    xbits = inputs.synthetic_x(m, k, dtype="f16")
    x = torch.from_numpy(xbits.view("int16")).to(dev).view(torch.float16)
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    call = Matmul(cabi, x, wbt, wst, out, m, k, n, cabi.CMK_F16, sh)
    log(f"[bench] prefill: M={m} K={k} N={n} f16, eager warm-up")
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    log(f"[bench] prefill: capturing {steps} launches")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(steps):
            call()
    graph.replay()
    torch.cuda.synchronize()
    ms = replay_timed(torch, cabi, graph, sh, steps, steps)
    flops = 2.0 * m * n * k
    t = ms / 1e3 / steps
    return {"m": m, "k": k, "n": n, "x_dtype": "f16", "ms_per_matmul": t * 1e3,
            "tflops": flops / t / 1e12, "frac_of_mfma_peak": flops / t / 1e12 / MFMA_F16_PEAK_TFLOPS,
            "gbs": alg_bytes(m, k, n, 2) / t / 1e9, "steps": steps}


# IQ2_XS, IQ2_S, IQ3_S: (ABI variant, bytes, scales per 256-weight block, the
# kernel that serves them at M=1)
VARIANTS = [("iq2_xs", 1, 64, 10,
             "cmk::iq2xxs_gemv_kernel<0, true, true, 1, false, false, 1, false> (one-row GEMV, IQ2_XS)"),
            ("iq2_s", 2, 72, 10,
             "cmk::iq2xxs_gemv_kernel<0, true, true, 1, false, false, 2, false> (one-row GEMV, IQ2_S)"),
            ("iq3_s", 3, 104, 6,
             "cmk::iq2xxs_gemv_kernel<0, true, true, 1, false, false, 3, false> (one-row GEMV, IQ3_S)")]


def bench_variants(pkg, torch, stream, steps, k=4096, n=14336):
    """The other formats' matmul at the config 1 gate shape (M=1, f32 x): one
    graph replay of `steps` launches over rotated weight copies per format."""
    cabi, inputs = pkg.cabi, pkg.inputs
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    bpr = math.ceil(k / 256)
    x = torch.from_numpy(inputs.synthetic_x(1, k)).to(dev)
    out = torch.empty((1, n), dtype=torch.float32, device=dev)
    res = {}
    for name, v, bpb, spb, fmt in VARIANTS:
        rng = np.random.default_rng(v)
        wb = rng.integers(0, 256, n * bpr * bpb, dtype=np.uint8)
        ws = rng.integers(0, 256, n * bpr * spb, dtype=np.uint8)
        ws[1::spb] = rng.integers(0x10, 0x20, n * bpr, dtype=np.uint8)  # finite d
        w_bytes = wb.size + ws.size
        copies = max(2, math.ceil(2 * MALL_BYTES / w_bytes))
        wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
        reps = [(wbt, wst)] + [(wbt.clone(), wst.clone()) for _ in range(copies - 1)]
        calls = [Matmul(cabi, x, r[0], r[1], out, 1, k, n, cabi.CMK_F32, sh, v) for r in reps]
        for c in calls:
            c()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                calls[i % copies]()
        graph.replay()
        torch.cuda.synchronize()
        us = replay_timed(torch, cabi, graph, sh, steps, steps) * 1e3 / steps
        alg = w_bytes + k * 4 + n * 4
        res[name] = {"k": k, "n": n, "m": 1, "mean_launch_us": us, "alg_bytes_per_launch": alg,
                     "gbs": alg / (us * 1e-6) / 1e9,
                     "frac_of_hbm_peak": alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                     "kernel": fmt,
                     "launches": steps}
        log(f"[bench] {name}: {us:.2f} us per launch, {res[name]['gbs']:.1f} GB/s")
        del graph, calls, reps
    return res


CONFIG4_SHAPES = [("q", 8192, 8192), ("k", 8192, 1024), ("v", 8192, 1024), ("o", 8192, 8192),
                  ("gate", 8192, 28672), ("up", 8192, 28672), ("down", 28672, 8192)]


def _timed_graph(torch, cabi, stream, sh, run, steps):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            run(i)
    graph.replay()
    torch.cuda.synchronize()
    return replay_timed(torch, cabi, graph, sh, steps, 4 * steps) * 1e3 / steps  # us per step


def bench_configs(pkg, torch, stream):
    """BASELINE config 2 (M in {4, 8, 16}, f32 x, %HBM; and W8A8 with int8
    activations, M in {4, 8, 16, 32} at N = 14336) and config 4 (the
    Llama-3-70B layer's seven projections back to back with f32 x: M=1 on the
    GEMV; M=128 rows staged as scaled f16 for the MFMA GEMM, then also with f16
    x given), over rotated weight copies."""
    cabi, inputs = pkg.cabi, pkg.inputs
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    res = {"config2": [], "config2_w8a8": [], "config4": {}}
    for k, n in ((4096, 4096), (4096, 14336)):
        wb, ws = inputs.synthetic_weights(n, k)
        w_bytes = wb.size + ws.size
        copies = max(2, math.ceil(2 * MALL_BYTES / w_bytes))
        wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
        reps = [(wbt, wst)] + [(wbt.clone(), wst.clone()) for _ in range(copies - 1)]
        for m in (4, 8, 16):
            x = torch.from_numpy(inputs.synthetic_x(m, k)).to(dev)
            out = torch.empty((m, n), dtype=torch.float32, device=dev)
            calls = [Matmul(cabi, x, r[0], r[1], out, m, k, n, cabi.CMK_F32, sh) for r in reps]
            for c in calls:
                c()
            us = _timed_graph(torch, cabi, stream, sh, lambda i: calls[i % copies](), 100)
            gbs = alg_bytes(m, k, n) / (us * 1e-6) / 1e9
            res["config2"].append({"m": m, "k": k, "n": n, "us": us, "gbs": gbs,
                                   "frac_of_hbm_peak": gbs / HBM_PEAK_GBS})
            log(f"[bench] config 2 m={m} k={k} n={n}: {us:.2f} us, {gbs:.1f} GB/s")
        for m in ((4, 8, 16, 32) if n == 14336 else ()):
            x = torch.from_numpy(inputs.synthetic_x(m, k)).to(dev)
            out = torch.empty((m, n), dtype=torch.float32, device=dev)
            calls = [Matmul(cabi, x, r[0], r[1], out, m, k, n, cabi.CMK_F32, sh,
                            mode=cabi.CMK_ACT_QUANT_W8A8) for r in reps]
            for c in calls:
                c()
            us = _timed_graph(torch, cabi, stream, sh, lambda i: calls[i % copies](), 100)
            gbs = alg_bytes(m, k, n) / (us * 1e-6) / 1e9
            path = cabi.matmul_path(cabi.CMK_F32, m, n, k, cabi.CMK_ACT_QUANT_W8A8)
            res["config2_w8a8"].append({"m": m, "k": k, "n": n, "us": us, "gbs": gbs,
                                        "path": path, "frac_of_hbm_peak": gbs / HBM_PEAK_GBS})
            log(f"[bench] config 2 W8A8 m={m} k={k} n={n} ({path}): {us:.2f} us, "
                f"{gbs:.1f} GB/s")
        del reps
    layer_w = sum(nn * math.ceil(kk / 256) * 66 for _, kk, nn in CONFIG4_SHAPES)
    copies = max(2, math.ceil(2 * MALL_BYTES / layer_w))
    weights = []
    for _, kk, nn in CONFIG4_SHAPES:
        wb, ws = inputs.synthetic_weights(nn, kk)
        wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
        weights.append([(wbt, wst)] + [(wbt.clone(), wst.clone()) for _ in range(copies - 1)])
    for m, dt in ((1, "f32"), (128, "f32"), (128, "f16")):
        calls = []
        for j, (_, kk, nn) in enumerate(CONFIG4_SHAPES):
            if dt == "f32":
                x = torch.from_numpy(inputs.synthetic_x(m, kk)).to(dev)
                xd = cabi.CMK_F32
            else:
                x = torch.from_numpy(inputs.synthetic_x(m, kk, dtype="f16").view("int16")).to(dev)
                x = x.view(torch.float16)
                xd = cabi.CMK_F16
            out = torch.empty((m, nn), dtype=torch.float32, device=dev)
            calls.append([Matmul(cabi, x, w[0], w[1], out, m, kk, nn, xd, sh) for w in weights[j]])

        def run(i):
            for per_proj in calls:
                per_proj[i % copies]()

        for i in range(copies):
            run(i)
        torch.cuda.synchronize()
        us = _timed_graph(torch, cabi, stream, sh, run, 20)
        xb = 4 if dt == "f32" else 2
        ab = sum(alg_bytes(m, kk, nn, xb) for _, kk, nn in CONFIG4_SHAPES)
        fl = sum(2.0 * m * kk * nn for _, kk, nn in CONFIG4_SHAPES)
        entry = {"m": m, "x_dtype": dt, "us_per_layer": us, "alg_bytes": ab,
                 "gbs": ab / (us * 1e-6) / 1e9, "tflops": fl / (us * 1e-6) / 1e12}
        entry["frac_of_hbm_peak"] = entry["gbs"] / HBM_PEAK_GBS
        entry["frac_of_mfma_peak"] = entry["tflops"] / MFMA_F16_PEAK_TFLOPS
        res["config4"][f"m{m}" + ("" if dt == "f32" else "_f16")] = entry
        log(f"[bench] config 4 m={m} ({dt}): {us:.1f} us per layer, {entry['gbs']:.1f} GB/s, "
            f"{entry['tflops']:.1f} TFLOP/s")
    return res


def bench_mlp_step(pkg, torch, stream, steps, k=4096, n=14336):
    """One Llama-3-8B MLP decode step with its data dependency: g = gate(x),
    h = silu(g) * up(x), y = down(h), over rotated weight copies; timed with the
    swiglu step in the up projection's epilogue (three launches) and, for
    comparison, composed with the swiglu kernel (four launches)."""
    cabi, inputs = pkg.cabi, pkg.inputs
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    step_w = sum(nn * math.ceil(kk / 256) * 66 for _, kk, nn in DECODE_SHAPES)
    copies = max(2, math.ceil(2 * MALL_BYTES / step_w))
    x = torch.from_numpy(inputs.synthetic_x(1, k)).to(dev)
    g = torch.empty((1, n), dtype=torch.float32, device=dev)
    u = torch.empty((1, n), dtype=torch.float32, device=dev)
    h = torch.empty((1, n), dtype=torch.float32, device=dev)
    y = torch.empty((1, k), dtype=torch.float32, device=dev)
    sets = []
    for name, kk, nn in DECODE_SHAPES:
        wb, ws = inputs.synthetic_weights(nn, kk)
        wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
        sets.append([(wbt, wst)] + [(wbt.clone(), wst.clone()) for _ in range(copies - 1)])
    calls = []
    for c in range(copies):
        (gw, gs), (uw, us), (dw, ds) = sets[0][c], sets[1][c], sets[2][c]
        calls.append((Matmul(cabi, x, gw, gs, g, 1, k, n, cabi.CMK_F32, sh),
                      Matmul(cabi, x, uw, us, u, 1, k, n, cabi.CMK_F32, sh),
                      Matmul(cabi, h, dw, ds, y, 1, n, k, cabi.CMK_F32, sh)))

    def run_composed(i):
        gate, up, down = calls[i % copies]
        gate()
        up()
        cabi.swiglu_raw(g.data_ptr(), u.data_ptr(), n, h.data_ptr(), cabi.CMK_F32, sh)
        down()

    def run_fused(i):
        gate, _, down = calls[i % copies]
        gate()
        uw, us = sets[1][i % copies]
        cabi.matmul_swiglu_raw(x.data_ptr(), cabi.CMK_F32, k, 1, uw.data_ptr(), uw.numel(),
                               us.data_ptr(), us.numel(), n, k, g.data_ptr(), n, h.data_ptr(),
                               stream=sh)
        down()

    def timed(run):
        for i in range(copies):
            run(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                run(i)
        graph.replay()
        torch.cuda.synchronize()
        return replay_timed(torch, cabi, graph, sh, steps, steps) * 1e3 / steps

    us_composed = timed(run_composed)
    us = timed(run_fused)
    step_bytes = sum(alg_bytes(1, kk, nn) for _, kk, nn in DECODE_SHAPES) + n * 8
    log(f"[bench] mlp step (gate, up, swiglu, down): {us_composed:.2f} us per step; "
        f"with silu(g)*u in up's epilogue: {us:.2f} us")
    return {"us_per_step": us, "launches_per_step": 3, "us_per_step_composed": us_composed,
            "launches_per_step_composed": 4, "alg_bytes_per_step": step_bytes,
            "gbs": step_bytes / (us * 1e-6) / 1e9, "steps": steps}


def bench_tp8_shards(pkg, torch, stream, steps=300):
    """One GPU's share of config 1 under 8-way tensor parallelism, at its real
    shape (M=1, f32 x): gate and up split by output rows (K=4096, N=1792 each)
    and down split by K (K=1792, N=4096, fp32 partials before the all-reduce).
    Rotated weight copies, one HIP graph per shape, mean launch time.  The
    collective itself is not measured (one GPU)."""
    cabi, inputs = pkg.cabi, pkg.inputs
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    res = {}
    for name, k, n in (("gate_or_up_1_of_8", 4096, 1792), ("down_1_of_8", 1792, 4096)):
        wb, ws = inputs.synthetic_weights(n, k)
        copies = max(2, math.ceil(2 * MALL_BYTES / (wb.size + ws.size)))
        wbt, wst = torch.from_numpy(wb).to(dev), torch.from_numpy(ws).to(dev)
        reps = [(wbt, wst)] + [(wbt.clone(), wst.clone()) for _ in range(copies - 1)]
        x = torch.from_numpy(inputs.synthetic_x(1, k)).to(dev)
        out = torch.empty((1, n), dtype=torch.float32, device=dev)
        calls = [Matmul(cabi, x, r[0], r[1], out, 1, k, n, cabi.CMK_F32, sh) for r in reps]
        for c in calls:
            c()
        torch.cuda.synchronize()
        us = _timed_graph(torch, cabi, stream, sh, lambda i: calls[i % copies](), steps)
        b = alg_bytes(1, k, n)
        res[name] = {"k": k, "n": n, "us_per_launch": us, "alg_bytes": b,
                     "gbs": b / (us * 1e-6) / 1e9}
        log(f"[bench] tp8 shard {name} (K={k} N={n}): {us:.2f} us per launch, "
            f"{res[name]['gbs']:.1f} GB/s")
        del reps, calls
    return res


def bench_gguf_split(pkg, torch, stream, steps, k=4096, n=14336):
    """GGUF (ggml) IQ2_XXS blocks of the gate matrix split into the reference's
    pair: bytes moved (read + written) per launch over its duration."""
    cabi = pkg.cabi
    dev = torch.device("cuda:0")
    sh = int(stream.cuda_stream)
    nb = n * math.ceil(k / 256)
    src = torch.randint(0, 256, (nb * 66,), dtype=torch.uint8, device=dev)
    wb = torch.empty(nb * 64, dtype=torch.uint8, device=dev)
    ws = torch.empty(nb * 2, dtype=torch.uint8, device=dev)

    def call():
        cabi.split_gguf_raw(src.data_ptr(), src.numel(), nb, cabi.CMK_IQ2_XXS, wb.data_ptr(),
                            wb.numel(), ws.data_ptr(), ws.numel(), sh)

    call()
    torch.cuda.synchronize()
    start, stop = cabi.Event(), cabi.Event()
    for _ in range(steps):  # untimed launches first: steady-state clocks
        call()
    start.record(sh)
    for _ in range(steps):
        call()
    stop.record(sh)
    torch.cuda.synchronize()
    us = start.elapsed_ms(stop) * 1e3 / steps
    moved = 2 * nb * 66
    log(f"[bench] gguf split: {us:.2f} us per launch, {moved / (us * 1e-6) / 1e9:.1f} GB/s")
    return {"variant": "iq2_xxs", "blocks": nb, "mean_launch_us": us, "bytes_moved": moved,
            "gbs": moved / (us * 1e-6) / 1e9, "launches": steps,
            "kernel": "cmk::gguf_split_kernel"}


def cpu_baseline(pkg, seconds):
    """The oracle (scalar restatement of the reference's CPU reference, OpenMP over
    outputs) on the same decode step; repeated until `seconds` of CPU time."""
    sys.path.insert(0, REPO)
    from oracle import oracle

    inputs = pkg.inputs
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or (os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or 1))
    data = []
    for _, k, n in DECODE_SHAPES:
        wb, ws = inputs.synthetic_weights(n, k)
        data.append((inputs.synthetic_x(1, k), k, n, wb, ws))
    step_bytes = sum(alg_bytes(1, k, n) for _, k, n in DECODE_SHAPES)
    reps = 0
    used = threads
    t0 = time.perf_counter()
    while True:
        for x, k, n, wb, ws in data:
            _, used = oracle.matmul_reference_mt(x, 1, n, k, wb, ws, threads=threads)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    # single-thread sample of one projection, for the per-core figure
    x, k, n, wb, ws = data[0]
    t1 = time.perf_counter()
    oracle.matmul_reference(x, 1, n, k, wb, ws)
    t1 = time.perf_counter() - t1
    return {
        "value": step_bytes * reps / el / 1e9,
        "unit": "GB/s",
        "cores": used,
        "kind": "port",
        "cpu_model": cpu_model(),
        "nproc": os.cpu_count(),
        "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
        "sample": (f"{reps} full decode steps (gate+up+down, M=1) in {el:.1f} s with the C "
                   f"oracle, OpenMP over outputs; 1-thread gate projection: "
                   f"{alg_bytes(1, k, n)/t1/1e9:.3f} GB/s"),
        "configs": cpu_config_samples(oracle, inputs, threads),
    }


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_config_samples(oracle, inputs, threads):
    """The oracle on bounded samples of BASELINE configs 0, 2, 3 and 4 (same
    threads): configs 0 and 2 whole, config 3 on 8 of its 512 rows (every row
    costs the same, so the rate is the full matmul's), config 4 at M=1 on the
    70B layer's gate projection.  Each figure is in the unit its config is
    quoted in on the GPU (GB/s at small m, GFLOP/s for the prefill)."""
    res = {}

    def run(name, m, k, n, rows=None, unit="GB/s"):
        wb, ws = inputs.synthetic_weights(n, k)
        mm = rows or m
        x = inputs.synthetic_x(mm, k)
        t = time.perf_counter()
        oracle.matmul_reference_mt(x, mm, n, k, wb, ws, threads=threads)
        t = time.perf_counter() - t
        if unit == "GB/s":
            v = alg_bytes(m, k, n) / t / 1e9
        else:
            v = 2.0 * mm * k * n / t / 1e9
        res[name] = {"m": m, "k": k, "n": n, "rows_run": mm, "seconds": round(t, 3),
                     "value": v, "unit": unit if unit == "GB/s" else "GFLOP/s"}

    run("config0", 1, 4096, 4096)
    run("config2_m8", 8, 4096, 14336)
    run("config3_m512", 512, 4096, 14336, rows=8, unit="GFLOP/s")
    run("config4_gate_m1", 1, 8192, 28672)
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=50)
    # The prefill line times one graph replay between host synchronisations; the
    # GPU clocks ramp back up over the first few milliseconds after the idle
    # gap, so the replay is made long (400 launches, about 25 ms) to report the
    # sustained rate rather than the ramp (50 launches read about 15 % slower).
    ap.add_argument("--prefill-steps", type=int, default=400)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the IQ2_XS / IQ2_S / IQ3_S lines")
    ap.add_argument("--variant-steps", type=int, default=200)
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the BASELINE config 2 and config 4 lines")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 256 MiB device copy (for rocprof counter calibration)")
    ap.add_argument("--traffic-summary", metavar="DIR",
                    help="summarise rocprofv3 FETCH_SIZE / WRITE_SIZE passes under DIR "
                         "into profiles/gemv_config1_traffic.json (no GPU needed)")
    ap.add_argument("--only", choices=["decode", "prefill", "read-floor", "variants", "configs"],
                    help="time one line only and print it (for profiling runs)")
    args = ap.parse_args()

    if args.traffic_summary:
        traffic_summary(args.traffic_summary, TRAFFIC_FILE)
        return

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} requested, but this build measures one GPU only "
              "(the IQ2_XXS path is single-GPU; see DESIGN.md for how it would shard).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    pkg = load_package()
    pkg.cabi.lib()

    if args.copy_calibration:
        n = 256 << 20
        a = torch.empty(n, dtype=torch.uint8, device="cuda:0")
        b = torch.empty(n, dtype=torch.uint8, device="cuda:0")
        a.fill_(1)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": n, "dispatches": 3}))
        return

    props = pkg.cabi.device_props()
    log(f"[bench] device: {props}")
    stream = torch.cuda.Stream()  # default priority
    if args.only:
        with torch.cuda.stream(stream):
            if args.only == "decode":
                res = bench_decode(pkg, torch, stream, args.steps, args.warmup)
            elif args.only == "prefill":
                res = bench_prefill(pkg, torch, stream, args.prefill_steps, 5)
            elif args.only == "variants":
                res = bench_variants(pkg, torch, stream, args.variant_steps)
            elif args.only == "configs":
                res = bench_configs(pkg, torch, stream)
            else:
                res = bench_read_floor(pkg, torch, stream, args.steps * len(DECODE_SHAPES))
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, **res}))
        return
    with torch.cuda.stream(stream):
        dec = bench_decode(pkg, torch, stream, args.steps, args.warmup)
        floor = bench_read_floor(pkg, torch, stream, args.steps * len(DECODE_SHAPES))
        prefill = (None if args.no_prefill
                   else bench_prefill(pkg, torch, stream, args.prefill_steps, 5))
        variants = (None if args.no_variants
                    else bench_variants(pkg, torch, stream, args.variant_steps))
        split = None if args.no_variants else bench_gguf_split(pkg, torch, stream, 50)
        shards = None if args.no_variants else bench_tp8_shards(pkg, torch, stream)
        refw = None if args.no_variants else bench_reference_workload(pkg, torch, stream)
        mlp = None if args.no_variants else bench_mlp_step(pkg, torch, stream, 300)
        configs = None if args.no_configs else bench_configs(pkg, torch, stream)
    torch.cuda.synchronize()
    value = dec["step_bytes"] * args.steps / (dec["ms"] / 1e3) / 1e9
    achieved = dec["per_launch_bytes"] / (dec["mean_launch_us"] * 1e-6) / 1e9
    traffic, traffic_source = load_traffic()
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dec["ms"] / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8-digit x iq2_xxs -> f32 (fp32 activations)",
        "data": "synthetic (seeded IQ2_XXS weights, N(0,1) fp32 activations)",
        "config": {"workload": "BASELINE config 1: Llama-3-8B MLP decode step at M=1 "
                               "(gate K=4096 N=14336, up K=4096 N=14336, down K=14336 N=4096)",
                   "m": 1, "launches_per_step": 3, "weight_copies_rotated": True},
        "frac_of_hbm_peak": value / HBM_PEAK_GBS,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_source": traffic_source,
                     "kernel": "cmk::iq2xxs_gemv_kernel<0, true, true, XT, false, false, 0, false> "
                               "(XT = 1 for K=4096, 2 for K=14336)",
                     "mean_launch_us": dec["mean_launch_us"],
                     "launch_us_over_replays": dec["launch_us_over_replays"],
                     "alg_bytes_per_launch": dec["per_launch_bytes"],
                     "read_floor": floor},
    }
    if prefill is not None:
        line["prefill_m512"] = prefill
    if variants is not None:
        line["variants_m1"] = variants
    if split is not None:
        line["gguf_split"] = split
    if shards is not None:
        line["tp8_shard_m1"] = shards
    if refw is not None:
        line["reference_bench_workload"] = refw
    if mlp is not None:
        line["mlp_step_m1"] = mlp
    if configs is not None:
        line["config2_small_m"] = configs["config2"]
        line["config2_w8a8_int8"] = configs["config2_w8a8"]
        line["config4_70b_layer"] = configs["config4"]
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(pkg, args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))


if __name__ == "__main__":
    main()
