#!/usr/bin/env python3
"""Benchmark of the quantized linear-layer hot path on one MI355X.

Workload (BASELINE.json metric "Q4_K matvec GB/s (% of HBM peak) at 8B
shapes"): one step = the M=1 decode matvecs of 8 distinct Llama-3-8B layers,
7 Q4_K projections each (attn q/k/v/output, ffn gate/up/down: 4096x4096,
1024x4096 x2, 4096x4096, 14336x4096 x2, 4096x14336), 981 MB of raw Q4_K
blocks per step - well above the 256 MB Infinity Cache, so every step reads
its weights from HBM.  Weights are seeded synthetic GGUF blocks (config 2
recipe), x ~ N(0,1) fp32, all resident in HBM before timing starts.  The step
is captured once as a HIP graph and replayed (one process, one GPU).

`value` = raw Q4_K bytes of K steps / their wall time (HIP events around the
replays).  `roofline` = the 14336x4096 matvec kernel, timed per launch with
HIP events on the launch stream while rotating over its 16 distinct copies.
`cpu_baseline` = the C/OpenMP transliteration of the reference's Numba loop
on one 14336x4096 matrix, timed on this host's cores in the same run.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_K matvec GB/s (% of HBM peak) at 8B shapes; 1B decode tokens/sec"
SHAPES_8B = [("attn_q", 4096, 4096), ("attn_k", 1024, 4096), ("attn_v", 1024, 4096),
             ("attn_output", 4096, 4096), ("ffn_gate", 14336, 4096),
             ("ffn_up", 14336, 4096), ("ffn_down", 4096, 14336)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4k_bytes(rows: int, cols: int) -> int:
    return rows * (cols // 256) * 144


def cpu_baseline(seconds: float) -> dict:
    """The reference's native-tier loop (C/OpenMP port) and its NumPy einsum
    path on one 14336x4096 Q4_K matrix (a bounded sample of the workload)."""
    import numpy as np

    from alpacca_amd import synth
    from oracle import cbaseline
    from oracle.qmatrix_ref import RefMatrix

    rows, cols = 14336, 4096
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=4242)
    ref = RefMatrix(data, "Q4_K", rows, cols)          # unpack: untimed
    x = synth.random_x(cols, seed=7)
    nbytes = q4k_bytes(rows, cols)
    loop = cbaseline.LoopMatvec(ref.q3, ref.d, ref.m)
    loop(x)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds * 0.6:
        loop(x)
        n += 1
    loop_s = (time.perf_counter() - t0) / n
    ref.matvec_ref(x)
    t0 = time.perf_counter()
    m = 0
    while time.perf_counter() - t0 < seconds * 0.4:
        ref.matvec_ref(x)
        m += 1
    np_s = (time.perf_counter() - t0) / m
    return {
        "value": round(nbytes / loop_s / 1e9, 3), "unit": "GB/s",
        "cores": cbaseline.cores(), "kind": "port",
        "sample": (f"one 14336x4096 Q4_K matvec (33,030,144 raw bytes), {n} calls of "
                   f"the C/OpenMP ({loop.isa}) transliteration of alpacca/kernels.py:49-69 "
                   f"over the reference's unpacked int8 codes; {loop_s * 1e3:.2f} ms/call"),
        "numpy_einsum": {"value": round(nbytes / np_s / 1e9, 3), "unit": "GB/s",
                         "ms_per_call": round(np_s * 1e3, 2), "calls": m,
                         "note": "qmatrix.py:160-171 order; einsum int8->f32 is single-threaded"},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--no-graph", action="store_true", help="time eager launches")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures a single GPU: --gpus {args.gpus} is not supported "
              "in this build (the hot path is one GPU's share; see DESIGN.md on sharding)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from alpacca_amd import synth
    from alpacca_amd.qmatrix import QuantMatrix

    torch.cuda.init()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}; building {args.layers} layers")

    mats = []
    for layer in range(args.layers):
        for si, (name, rows, cols) in enumerate(SHAPES_8B):
            data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=100 * layer + si)
            mats.append((name, layer, QuantMatrix(data, "Q4_K", rows, cols), rows, cols))
    step_bytes = sum(q4k_bytes(r, c) for _, _, _, r, c in mats)
    xs = {c: torch.from_numpy(synth.random_x(c, seed=c)).to(dev) for c in {4096, 14336}}
    ys = [torch.empty(r, dtype=torch.float32, device=dev) for _, _, _, r, _ in mats]
    log(f"uploaded {len(mats)} matrices, {step_bytes / 1e6:.1f} MB per step")

    stream = torch.cuda.Stream(dev)  # default priority

    def step(s) -> None:
        h = s.cuda_stream
        for (_, _, qm, _, cols), y in zip(mats, ys):
            qm.matvec_device(xs[cols].data_ptr(), y.data_ptr(), h)

    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            step(stream)
    torch.cuda.synchronize()

    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            step(stream)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for _ in range(args.warmup):
                graph.replay()
        torch.cuda.synchronize()

    # ---- timed region: K steps ----
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(args.steps):
            if graph is not None:
                graph.replay()
            else:
                step(stream)
        end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    value = step_bytes * args.steps / (total_ms * 1e-3) / 1e9
    log(f"{args.steps} steps: {ms_per_step:.4f} ms/step, {value:.1f} GB/s")

    # ---- dominant kernel: 14336x4096, per-launch HIP events, 16 copies ----
    gate = [(qm, y) for (name, _, qm, _, _), y in zip(mats, ys) if name in ("ffn_gate", "ffn_up")]
    reps = max(4, args.steps // 2)
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(reps * len(gate))]
    with torch.cuda.stream(stream):
        for qm, y in gate:
            qm.matvec_device(xs[4096].data_ptr(), y.data_ptr(), stream.cuda_stream)
        i = 0
        for _ in range(reps):
            for qm, y in gate:
                pairs[i][0].record(stream)
                qm.matvec_device(xs[4096].data_ptr(), y.data_ptr(), stream.cuda_stream)
                pairs[i][1].record(stream)
                i += 1
    torch.cuda.synchronize()
    durs = np.array([a.elapsed_time(b) for a, b in pairs]) * 1e3  # us
    kbytes = q4k_bytes(14336, 4096)
    achieved = kbytes / (durs.mean() * 1e-6) / 1e9
    log(f"14336x4096 Q4_K matvec: mean {durs.mean():.2f} us, median {np.median(durs):.2f} us "
        f"-> {achieved:.1f} GB/s")

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline ({args.cpu_seconds:.0f} s budget)")
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} cores")

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded GGUF Q4_K blocks (config 2 recipe), x ~ N(0,1) fp32",
        "config": {
            "workload": (f"Q4_K decode matvec (M=1) over {args.layers} distinct Llama-3-8B "
                         "layers x 7 projections (4096x4096, 1024x4096 x2, 4096x4096, "
                         "14336x4096 x2, 4096x14336), HIP-graph replay"
                         + ("" if graph is not None else " disabled (eager)")),
            "bytes_per_step": step_bytes,
            "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "k_matvec<Q4K,4,1> 14336x4096",
            "bytes_per_launch": kbytes, "mean_us": round(float(durs.mean()), 3),
            "median_us": round(float(np.median(durs)), 3),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
