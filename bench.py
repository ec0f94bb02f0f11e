#!/usr/bin/env python3
"""Benchmark of the quantized linear-layer hot path on one MI355X.

Workload (BASELINE.json metric "Q4_K matvec GB/s (% of HBM peak) at 8B
shapes"): one step = the M=1 decode matvecs of 8 distinct Llama-3-8B layers,
7 Q4_K projections each (attn q/k/v/output 4096x4096, 1024x4096 x2,
4096x4096; ffn gate/up 14336x4096 x2, down 4096x14336) = 981,467,136 raw
bytes per step, well above the 256 MB Infinity Cache, so every step streams
its weights from HBM.  The launches follow a decode layer's dependency
structure: q/k/v share one input and run as one fused launch, gate/up as
another, output and down alone (4 launches per layer).  Weights are seeded
synthetic GGUF blocks (config 2 recipe), x ~ N(0,1) fp32, all resident in HBM
before timing starts.  The step is captured once as a HIP graph and replayed.

`value` = raw Q4_K bytes of K steps / their wall time (HIP events on the
launch stream).  `roofline` = the dominant kernel, the fused ffn_gate+ffn_up
launch (66 MB, 54 % of a step's bytes): 12 rounds over the 8 layers'
launches captured as one graph, replayed between two HIP events on the
launch stream; the average launch duration is the elapsed time over the 96
launches (graph replay leaves no gap between kernels, so this agrees with
the profiler's kernel durations).  `traffic` is read from the committed
rocprofv3 counter runs of the same launches (profiles/).  `cpu_baseline` =
the C/OpenMP transliteration of the reference's Numba loop on one 14336x4096
matrix, on this host's cores, same run.

`roofline.read_ceiling` = the same byte count read by the library's bare
streaming-read kernel (aq_stream_read) over a sweep of launch shapes: what
one launch of that size can read from HBM on this part, which the datasheet
8 TB/s is not; `frac_of_read_ceiling` = achieved / that rate.

Further legs in the same JSON line: `matvec_configs` (every M=1 shape of
configs 1-3, each rotating over >= 512 MB of HBM copies), `small_batch`
(matmul_t with 1, 4 and 16 rows of X on the integer kernel), `prefill`
(config 4) and `decode_1b` (config 5).

`--decode-ops` times each op type of the config-5 decode step on its own
inside HIP graphs.  `--calibrate` instead times PyTorch's own copy and sum kernels on buffers of
known size (the streaming ceiling of this GPU, and the reference point used to
scale rocprofv3 FETCH_SIZE / WRITE_SIZE readings).  `--summarize DB` prints
the summary of a rocprofv3 results database of a run of this script.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

HBM_PEAK_GBS = 8000.0
METRIC = "Q4_K matvec GB/s (% of HBM peak) at 8B shapes; 1B decode tokens/sec"
SHAPES_8B = [("attn_q", 4096, 4096), ("attn_k", 1024, 4096), ("attn_v", 1024, 4096),
             ("attn_output", 4096, 4096), ("ffn_gate", 14336, 4096),
             ("ffn_up", 14336, 4096), ("ffn_down", 4096, 14336)]
ROOFLINE_REPS = 12
ROOFLINE_REPLAYS = 5  # timed replays of the roofline leg's graph
TRAFFIC_PROFILE = Path(__file__).resolve().parent / "profiles" / "k_matvec_i8_q4k_gate_up_traffic.json"
# the gate/up launch (gate and up as one matrix): the one-matrix kernel, Q4_K
# units, one row per iteration, three rows in flight, one step per row, 512
# threads, plain x, one row per wave
DOMINANT = "k_matvec_i8_one<aq::UQ4K, 1, 3, true, 512, 0, false>"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4k_bytes(rows: int, cols: int) -> int:
    return rows * (cols // 256) * 144


def host_facts() -> dict:
    """The CPU the baseline legs ran on: model, the cores this process may use,
    NumPy and its BLAS, and whether the reference's Numba tier could run."""
    import importlib.util
    import os
    import platform

    import numpy as np
    model = platform.processor() or "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    blas = None
    try:
        from threadpoolctl import threadpool_info
        blas = [{"api": i.get("internal_api"), "threads": i.get("num_threads")}
                for i in threadpool_info() if i.get("user_api") == "blas"]
    except Exception:  # pragma: no cover - optional
        pass
    numba = importlib.util.find_spec("numba") is not None
    return {"cpu_model": model, "cores": len(os.sched_getaffinity(0)),
            "numpy": np.__version__, "blas": blas,
            "numba": ("installed" if numba else
                      "not installed: alpacca/kernels.py:76-86 would report the Numba tier "
                      "unavailable, so the reference runs its NumPy path; the C/OpenMP port "
                      "of kernels.py:49-69 stands in for the Numba leg")}


def _time_calls(fn, seconds: float, min_calls: int = 2):
    fn()
    n, t0 = 0, time.perf_counter()
    while n < min_calls or time.perf_counter() - t0 < seconds:
        fn()
        n += 1
    return (time.perf_counter() - t0) / n, n


def cpu_config_legs(tensors_1b=None, hp_1b=None) -> dict:
    """Bounded CPU samples of configs 1, 4 and 5 on this host, with the
    oracle's restatements of the reference paths: C1 Q8_0 2048x2048 matvec
    (NumPy einsum order of qmatrix.py:160-171, and the C/OpenMP port of the
    Numba loop kernels.py:49-69); C4 matmul_t at M = 512 (qmatrix.py:196-211:
    f32 row tiles times X through NumPy/BLAS on every core); C5 the decode
    step of the synthetic 1B model (model.py:520-555, both matvec tiers) at
    positions 2048.. with a KV cache of 2048 seeded positions, 8 steps each
    (tests/bench.py:82-95 times decode steps the same way)."""
    import numpy as np

    from alpacca_amd import synth
    from oracle import cbaseline
    from oracle.qmatrix_ref import RefMatrix
    out: dict = {}
    raw = synth.random_matrix_bytes("Q8_0", 2048, 2048, seed=4096)
    ref = RefMatrix(raw, "Q8_0", 2048, 2048)
    x = synth.random_x(2048, seed=2048)
    loop = cbaseline.LoopMatvec(ref.q3, ref.d, ref.m)
    t_np, n_np = _time_calls(lambda: ref.matvec_ref(x), 1.0)
    t_c, n_c = _time_calls(lambda: loop(x), 1.0, 20)
    out["C1_q8_0_2048x2048_matvec"] = {
        "bytes": len(raw),
        "numpy_einsum": {"GBps": round(len(raw) / t_np / 1e9, 3), "us_per_call": round(t_np * 1e6, 1),
                         "calls": n_np},
        "c_port_of_numba_loop": {"GBps": round(len(raw) / t_c / 1e9, 3),
                                 "us_per_call": round(t_c * 1e6, 1), "calls": n_c}}
    log(f"cpu C1: numpy {len(raw) / t_np / 1e9:.2f} GB/s, C port {len(raw) / t_c / 1e9:.1f} GB/s")
    rows = []
    for dtype, M, n, k, _ in PREFILL_CASES:
        if any(r["case"].startswith(f"{dtype} X {M}x{k} W {n}x{k}") for r in rows):
            continue
        mref = RefMatrix(synth.random_matrix_bytes(dtype, n, k, seed=n + k), dtype, n, k)
        X = synth.random_x(k, seed=5, batch=M)
        t, calls = _time_calls(lambda: mref.matmul_t_ref(X), 1.0)
        flops = 2 * M * n * k
        rows.append({"case": f"{dtype} X {M}x{k} W {n}x{k}", "TFLOP/s": round(flops / t / 1e12, 3),
                     "ms_per_call": round(t * 1e3, 1), "calls": calls})
        log(f"cpu C4 {dtype} {M}x{n}x{k}: {flops / t / 1e12:.3f} TFLOP/s")
        del mref
    out["C4_matmul_t_ref"] = rows
    if tensors_1b is not None:
        from oracle.model_ref import RefModel
        t0 = time.perf_counter()
        rm = RefModel(hp_1b, tensors_1b, n_ctx=DECODE_PROMPT + DECODE_GEN, fast=True)
        build_s = time.perf_counter() - t0
        rng = np.random.default_rng(2048)
        for li in range(hp_1b.n_layer):
            shape = (DECODE_PROMPT, hp_1b.n_kv, hp_1b.head_dim)
            rm.cache_k[li][:DECODE_PROMPT] = rng.standard_normal(shape, dtype=np.float32)
            rm.cache_v[li][:DECODE_PROMPT] = rng.standard_normal(shape, dtype=np.float32)
        toks = [int(t) for t in rng.integers(0, hp_1b.n_vocab, 8)]

        def steps():
            rm.n_past = DECODE_PROMPT
            t0 = time.perf_counter()
            for t in toks:
                rm.forward(t)
            return (time.perf_counter() - t0) / len(toks)
        fast_s = steps()
        mats = [m for ly in rm.layers for m in ly.values() if hasattr(m, "_loop")]
        for m in mats + [rm.output]:
            m._loop = None
        numpy_s = steps()
        out["C5_decode_1b"] = {
            "context": DECODE_PROMPT, "steps": len(toks),
            "numpy_path_tokens_per_s": round(1 / numpy_s, 3),
            "c_port_of_numba_loop_tokens_per_s": round(1 / fast_s, 3),
            "oracle_build_s": round(build_s, 1),
            "note": "RefModel.forward (oracle/model_ref.py, model.py:520-555): matvecs through "
                    "the NumPy einsum path, then through the C port of the Numba loop; "
                    "KV cache of 2048 seeded positions"}
        log(f"cpu C5: numpy {1 / numpy_s:.2f} tok/s, C port {1 / fast_s:.2f} tok/s "
            f"(oracle build {build_s:.0f} s)")
        del rm
    return out


def cpu_baseline(seconds: float, tensors_1b=None, hp_1b=None) -> dict:
    """The reference's native-tier loop (C/OpenMP port) and its NumPy einsum
    path on one 14336x4096 Q4_K matrix (a bounded sample of the workload),
    then the config 1, 4 and 5 legs (cpu_config_legs) and the host facts."""
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
    del ref, loop
    return {
        "value": round(nbytes / loop_s / 1e9, 3), "unit": "GB/s",
        "cores": cbaseline.cores(), "kind": "port",
        "sample": (f"one 14336x4096 Q4_K matvec (33,030,144 raw bytes), {n} calls of "
                   f"the C/OpenMP transliteration of alpacca/kernels.py:49-69 "
                   f"over the reference's unpacked int8 codes; {loop_s * 1e3:.3f} ms/call"),
        "numpy_einsum": {"value": round(nbytes / np_s / 1e9, 3), "unit": "GB/s",
                         "ms_per_call": round(np_s * 1e3, 2), "calls": m, "cores": 1,
                         "note": "qmatrix.py:160-171 order; einsum int8->f32 is single-threaded"},
        "host": host_facts(),
        "configs": cpu_config_legs(tensors_1b, hp_1b),
    }


# configs 1-3 of BASELINE.json: (config, dtype, rows, cols) of the M=1 matvecs
MATVEC_CONFIGS = [("C1", "Q8_0", 2048, 2048),
                  ("C2", "Q4_K", 2048, 2048), ("C2", "Q4_K", 512, 2048),
                  ("C2", "Q4_K", 8192, 2048), ("C2", "Q4_K", 2048, 8192),
                  ("C3", "Q5_K", 4096, 4096), ("C3", "Q5_K", 1024, 4096),
                  ("C3", "Q5_K", 14336, 4096), ("C3", "Q6_K", 4096, 14336),
                  ("C3", "Q6_K", 128256, 4096),
                  # Q4_0, the other 18-byte-block format the north star names
                  ("Q4_0", "Q4_0", 4096, 4096), ("Q4_0", "Q4_0", 14336, 4096)]
ROTATE_BYTES = 512e6  # distinct HBM copies per timed shape: twice the 256 MB Infinity Cache


def _graph_time(stream, fn, launches: int) -> float:
    """Mean microseconds per launch of fn(i), i < launches, captured as one HIP
    graph on `stream` and replayed between two HIP events on that stream
    (best of three replays after a warmup replay)."""
    import torch
    with torch.cuda.stream(stream):
        fn(0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(launches):
            fn(i)
    with torch.cuda.stream(stream):
        g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            a.record(stream)
            g.replay()
            b.record(stream)
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) * 1e3 / launches)
    return best


READ_SWEEP = ((2048, 1), (2048, 2), (2048, 4), (4096, 1), (4096, 2), (4096, 4),
              (8192, 1), (8192, 2))  # (waves, rows in flight per wave)


def read_ceiling_leg(dev, stream, nbytes: int, row_bytes: int = 2304) -> dict:
    """What one launch can read from HBM on this part at the dominant
    launch's byte count: the library's streaming-read kernel (aq_stream_read,
    rows of row_bytes strided over the waves as the decode matvec reads them)
    over READ_SWEEP's launch shapes, rotating over distinct buffers of
    >= 700 MB in a HIP graph; the fastest shape is the ceiling."""
    import ctypes

    import torch

    from alpacca_amd import _lib
    lib = _lib.ensure_device()
    copies = max(4, -(-int(700e6) // nbytes))
    bufs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev) for _ in range(copies)]
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    rows = nbytes // row_bytes
    h = ctypes.c_void_p(stream.cuda_stream)
    shapes = []
    for waves, inflight in READ_SWEEP:
        us = _graph_time(stream, lambda i: _lib.check(lib.aq_stream_read(
            ctypes.c_void_p(bufs[i % copies].data_ptr()), rows, row_bytes, waves, inflight,
            ctypes.c_void_p(sink.data_ptr()), h)), 2 * copies)
        shapes.append({"waves": waves, "inflight": inflight, "us": round(us, 2),
                       "GB/s": round(rows * row_bytes / us / 1e3, 1)})
        log(f"read ceiling {nbytes / 1e6:.1f} MB, {waves} waves x {inflight} rows in flight: "
            f"{us:.2f} us, {rows * row_bytes / us / 1e3:.0f} GB/s")
    del bufs
    torch.cuda.empty_cache()
    best = min(shapes, key=lambda r: r["us"])
    return {"kernel": "aq_stream_read (rows strided over waves, 16 B per lane per load)",
            "bytes": rows * row_bytes, "us": best["us"], "GB/s": best["GB/s"],
            "frac_of_peak": round(best["GB/s"] / HBM_PEAK_GBS, 4),
            "best_shape": {"waves": best["waves"], "inflight": best["inflight"]},
            "sweep": shapes}


def _copies(raw: bytes, dtype: str, rows: int, cols: int) -> list:
    from alpacca_amd.qmatrix import QuantMatrix
    n = max(2, -(-int(ROTATE_BYTES) // len(raw)))
    return [QuantMatrix(raw, dtype, rows, cols) for _ in range(n)]


def matvec_configs_leg(dev, stream) -> list:
    """Configs 1-3: the M=1 decode matvec (default integer kernel) of every
    config shape, one matrix per launch, rotating over distinct HBM copies
    of >= 512 MB in a HIP graph; GB/s = raw quantized bytes / launch time,
    frac against the 8 TB/s HBM peak."""
    import torch

    from alpacca_amd import synth
    out = []
    for cfg, dtype, rows, cols in MATVEC_CONFIGS:
        raw = synth.random_matrix_bytes(dtype, rows, cols, seed=rows + cols)
        mats = _copies(raw, dtype, rows, cols)
        x = torch.from_numpy(synth.random_x(cols, seed=cols)).to(dev)
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        n = len(mats)
        us = _graph_time(stream, lambda i: mats[i % n].matvec_device(
            x.data_ptr(), y.data_ptr(), stream.cuda_stream), max(2 * n, 24))
        gbs = len(raw) / (us * 1e-6) / 1e9
        log(f"{cfg} {dtype} {rows}x{cols} ({len(raw):,} B, {mats[0].layout}): {us:.2f} us, "
            f"{gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.3f} of peak), {n} copies")
        out.append({"config": cfg, "dtype": dtype, "shape": [rows, cols], "layout": mats[0].layout,
                    "bytes": len(raw), "us_per_launch": round(us, 3), "GBps": round(gbs, 1),
                    "frac_peak": round(gbs / HBM_PEAK_GBS, 4), "copies": n})
        del mats
        torch.cuda.empty_cache()
    return out


# (--small-batch-formats) small batches of the other formats the exact fp16
# kernels take: below 9 rows the integer kernel, from 9 rows the exact
# kernels' 16- and 32-row tiles, from 33 rows their 64 x 256 tiles
SMALL_FORMAT_CASES = [("Q6_K", 14336, 4096), ("Q6_K", 4096, 14336), ("Q8_0", 14336, 4096),
                      ("Q4_0", 14336, 4096), ("Q5_1", 14336, 4096)]
SMALL_FORMAT_MS = (8, 16, 32, 63)


def small_batch_formats_leg(dev, stream) -> list:
    """matmul_t at the default precision with 8, 16, 32 and 63 rows of X
    against the SMALL_FORMAT_CASES matrices, rotating copies in a HIP graph
    (the method of small_batch_leg)."""
    import torch

    from alpacca_amd import synth
    out = []
    for dtype, rows, cols in SMALL_FORMAT_CASES:
        raw = synth.random_matrix_bytes(dtype, rows, cols, seed=78)
        mats = _copies(raw, dtype, rows, cols)
        n = len(mats)
        for M in SMALL_FORMAT_MS:
            X = torch.from_numpy(synth.random_x(cols, seed=M, batch=M)).to(dev)
            Y = torch.empty((M, rows), dtype=torch.float32, device=dev)
            us = _graph_time(stream, lambda i: mats[i % n].matmul_t_device(
                X.data_ptr(), M, Y.data_ptr(), stream.cuda_stream, "auto"), max(2 * n, 16))
            log(f"small batch {dtype} {rows}x{cols} M={M}: {us:.2f} us, "
                f"{len(raw) / (us * 1e-6) / 1e9:.0f} GB/s of weights")
            out.append({"dtype": dtype, "rows": rows, "cols": cols, "M": M,
                        "us_per_call": round(us, 2)})
        del mats
        torch.cuda.empty_cache()
    return out


def small_batch_leg(dev, stream) -> list:
    """matmul_t with 1, 4, 8, 16, 32 and 48 rows of X against Q4_K 14336x4096
    (the 8B gate shape) at the default precision ("auto", float32 accuracy:
    below 3 rows the integer decode kernel with several x vectors sharing
    one weight stream, from 3 rows the exact-integer fp16 MFMA kernel),
    rotating copies in a HIP graph; GB/s of weight bytes per call and
    microseconds per x vector."""
    import torch

    from alpacca_amd import synth
    rows, cols = 14336, 4096
    raw = synth.random_matrix_bytes("Q4_K", rows, cols, seed=77)
    mats = _copies(raw, "Q4_K", rows, cols)
    n = len(mats)
    out = []
    for M in (1, 4, 8, 16, 32, 48):
        X = torch.from_numpy(synth.random_x(cols, seed=M, batch=M)).to(dev)
        Y = torch.empty((M, rows), dtype=torch.float32, device=dev)
        us = _graph_time(stream, lambda i: mats[i % n].matmul_t_device(
            X.data_ptr(), M, Y.data_ptr(), stream.cuda_stream, "auto"), max(2 * n, 16))
        gbs = len(raw) / (us * 1e-6) / 1e9
        log(f"small batch Q4_K {rows}x{cols} M={M}: {us:.2f} us, {gbs:.0f} GB/s of weights, "
            f"{us / M:.2f} us per x vector")
        out.append({"M": M, "us_per_call": round(us, 2), "weight_GBps": round(gbs, 1),
                    "us_per_vector": round(us / M, 3)})
    del mats
    torch.cuda.empty_cache()
    return out


# (dtype, M, rows, cols, precision): config 4 - the two Q4_K shapes on the
# bf16 path and on the default float32-accuracy path ("auto"), and the Q8_0
# variant with int8 activations as configured (per-32 absmax-quantized X),
# beside the same Q8_0 matrix on the bf16 path and at the default precision
PREFILL_CASES = [("Q4_K", 512, 14336, 4096, "bf16"), ("Q4_K", 512, 4096, 14336, "bf16"),
                 ("Q4_K", 512, 14336, 4096, "auto"), ("Q4_K", 512, 4096, 14336, "auto"),
                 ("Q8_0", 512, 4096, 4096, "int8"), ("Q8_0", 512, 4096, 4096, "bf16"),
                 ("Q8_0", 512, 4096, 4096, "auto")]
# dense MFMA peaks (TOP/s for int8).  "auto" (float32 accuracy) runs on the
# fp16 matrix cores with x in two fp16 pieces: two MFMA flops per useful flop,
# priced against the fp16 peak (frac_peak of the useful flops, and the MFMA
# work's own fraction beside it)
PEAK_TFLOPS = {"bf16": 2500.0, "int8": 5000.0, "auto": 2500.0, "fp32": 2500.0}
MFMA_FLOPS_PER_FLOP = {"bf16": 1, "int8": 1, "auto": 2, "fp32": 2}
# (--formats-only) matmul_t at float32 accuracy for every format the exact
# fp16 kernels take: "auto" (split over workgroups where the tiles are few)
# and "fp32" (no split: the batched prefill step's precision); the 1B
# model's Q6_K v and ffn_down shapes at its 2048-token prefill, and
# 4096x4096 at M = 512 for the others
FORMAT_CASES = [(d, M, r, c, p) for d, M, r, c in
                [("Q5_K", 512, 14336, 4096), ("Q6_K", 2048, 2048, 8192), ("Q6_K", 2048, 512, 2048),
                 ("Q8_0", 512, 4096, 4096), ("Q4_0", 512, 4096, 4096), ("Q4_1", 512, 4096, 4096),
                 ("Q5_0", 512, 4096, 4096), ("Q5_1", 512, 4096, 4096)]
                for p in ("auto", "fp32")]


def prefill_leg(dev, stream, reps: int = 20, cases=None) -> list:
    """Config 4: batched prefill Y = X W^T at M = 512 for each PREFILL_CASES
    row, timed with HIP events on the launch stream over `reps` calls after a
    warmup (each call includes its X conversion or quantization launch);
    2*M*N*K flops per call against the dense MFMA peak of the precision
    (int8: TOP/s against 5.0 POP/s; "auto", the float32-accuracy default:
    against the fp16 peak its matrix cores run at, two MFMA flops per flop)."""
    import torch

    from alpacca_amd import synth
    from alpacca_amd.qmatrix import QuantMatrix
    out = []
    for dtype, M, rows, cols, prec in cases or PREFILL_CASES:
        qm = QuantMatrix(synth.random_matrix_bytes(dtype, rows, cols, seed=rows + cols),
                         dtype, rows, cols)
        X = torch.from_numpy(synth.random_x(cols, seed=5, batch=M)).to(dev)
        Y = torch.empty((M, rows), dtype=torch.float32, device=dev)
        h = stream.cuda_stream
        with torch.cuda.stream(stream):
            for _ in range(3):
                qm.matmul_t_device(X.data_ptr(), M, Y.data_ptr(), h, prec)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            a.record(stream)
            for _ in range(reps):
                qm.matmul_t_device(X.data_ptr(), M, Y.data_ptr(), h, prec)
            b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps
        flops = 2 * M * rows * cols
        tf = flops / (us * 1e-6) / 1e12
        log(f"prefill {dtype} {prec} M={M} {rows}x{cols}: {us:.1f} us/call, {tf:.1f} T(FL)OP/s")
        out.append({"case": f"{dtype} X {M}x{cols} W {rows}x{cols}", "precision": prec,
                    "us_per_call": round(us, 2), "flops": flops,
                    "TFLOP/s": round(tf, 2), "frac_peak": round(tf / PEAK_TFLOPS[prec], 4),
                    "peak": PEAK_TFLOPS[prec], "mfma_flops_per_flop": MFMA_FLOPS_PER_FLOP[prec],
                    "frac_peak_mfma_work": round(tf * MFMA_FLOPS_PER_FLOP[prec]
                                                 / PEAK_TFLOPS[prec], 4)})
        del qm, X, Y
    return out

DECODE_PROMPT, DECODE_GEN = 2048, 256
GOLDEN_DECODE = Path(__file__).resolve().parent / "tests" / "golden" / "decode_1b_greedy.json"
GOLDEN_DECODE_PENALTY = GOLDEN_DECODE.with_name("decode_1b_greedy_penalty.json")


def _golden_match(path: Path, toks: list) -> bool | None:
    try:
        gold = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    if gold.get("n_prompt") != DECODE_PROMPT or gold.get("n_gen") != DECODE_GEN:
        return None
    return gold["tokens"] == toks


def decode_leg(hp=None, tensors=None) -> dict:
    """Config 5: greedy decode on the synthetic Llama-3.2-1B-shaped model
    (alpacca_amd.model.synthetic_llama_1b, seed 0): a 2048-token seeded
    prompt fills the fp32 KV cache, then 256 greedy tokens; each token is
    one HIP-graph replay of the device-resident step.  The prompt runs
    through the batched step (fp32 MFMA matmuls, one 2048-token chunk;
    bit-identical to the reference's 256-token chunks); the first token is
    the argmax of its logits, and each of the other 255 is one graph
    replay.  tokens/s = 255 /
    elapsed time of those replays (HIP events on the launch stream).  The
    tokens are compared with the oracle's committed trace when present.
    A second run uses the reference benchmark's own selection
    (tests/bench.py:78-90: temperature-0 Sampler, repetition penalty 1.1 over
    the last 64 accepted tokens, sample.py:31-45), reported as "penalized".
    prefill_ms is the first prefill of the process's model, timed like the
    reference's bench (tests/bench.py:82-84: one call, host clock), so it
    includes first-launch costs; prefill_ms_second_run is the second run's
    prefill of the same prompt on the emptied cache."""
    import numpy as np

    from alpacca_amd.model import Model, synthetic_llama_1b
    if tensors is None:
        hp, tensors = synthetic_llama_1b(seed=0)
    model = Model(hp, tensors, n_ctx=DECODE_PROMPT + DECODE_GEN)
    layer_bytes = sum(len(t.data) for n, t in tensors.items()
                      if t.dtype != "F32" and n.startswith("blk."))
    head_bytes = len(tensors["output.weight"].data)
    prompt = [int(t) for t in np.random.default_rng(2048).integers(0, hp.n_vocab, DECODE_PROMPT)]
    timing: dict = {}
    toks = model.generate_greedy(prompt, DECODE_GEN, graph=True, timing=timing)
    tps = timing["steps"] / (timing["gen_ms"] * 1e-3)
    # KV bytes read per step at position p: layers * 2 * n_kv * head_dim * 4 * (p + 1)
    kv_per_pos = hp.n_layer * 2 * hp.n_kv * hp.head_dim * 4
    first = DECODE_PROMPT - 1
    kv_avg = kv_per_pos * (sum(range(first + 1, first + DECODE_GEN + 1)) / DECODE_GEN)
    bytes_tok = layer_bytes + head_bytes + kv_avg
    match = _golden_match(GOLDEN_DECODE, toks)
    log(f"decode 1B: prefill {DECODE_PROMPT} tokens {timing['prefill_ms']:.1f} ms; "
        f"{timing['gen_ms']:.2f} ms for {timing['steps']} steps -> {tps:.1f} tok/s, "
        f"{bytes_tok * tps / 1e9:.0f} GB/s; tokens match oracle: {match}")
    pt: dict = {}
    ptoks = model.generate_greedy(prompt, DECODE_GEN, graph=True, timing=pt,
                                  repeat_penalty=1.1, repeat_last_n=64)
    ptps = pt["steps"] / (pt["gen_ms"] * 1e-3)
    pmatch = _golden_match(GOLDEN_DECODE_PENALTY, ptoks)
    log(f"decode 1B, repetition penalty 1.1 / 64: {ptps:.1f} tok/s; "
        f"tokens match oracle: {pmatch}; its prefill (the same prompt, second run) "
        f"{pt['prefill_ms']:.1f} ms")
    return {"tokens_per_s": round(tps, 1), "ms_per_token": round(timing["gen_ms"] / timing["steps"], 4),
            "prefill_ms": round(timing["prefill_ms"], 2),
            "prefill_tokens_per_s": round(DECODE_PROMPT / (timing["prefill_ms"] * 1e-3), 1),
            # the second run's prefill of the same prompt (emptied cache; kernels
            # loaded and buffers allocated by the first): the steady-state figure
            "prefill_ms_second_run": round(pt["prefill_ms"], 2),
            "bytes_per_token": int(bytes_tok), "weight_bytes_per_token": layer_bytes + head_bytes,
            "achieved_GBps": round(bytes_tok * tps / 1e9, 1),
            "hbm_fraction": round(bytes_tok * tps / 1e9 / HBM_PEAK_GBS, 4),
            "prompt": DECODE_PROMPT, "generated": DECODE_GEN,
            "tokens_match_oracle": match, "first_tokens": toks[:8],
            "penalized": {"tokens_per_s": round(ptps, 1), "repeat_penalty": 1.1,
                          "repeat_last_n": 64, "tokens_match_oracle": pmatch,
                          "selection": "tests/bench.py:78-90 (Sampler, temperature 0)"},
            "model": "synthetic Llama-3.2-1B shape (16 layers, 2048 hidden, 32/8 heads, FFN 8192, "
                     "vocab 128256), Q4_K + Q6_K (attn_v, 8 ffn_down, output), fp32 KV"}


DROP_IN_ORDER = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


def drop_in_leg(hp, tensors, tokens: int = 20) -> dict:
    """What an unchanged reference model.py pays for its matvecs through the
    drop-in: per token it calls QuantMatrix.matvec on host (NumPy) arrays 113
    times - q, k, v, o, gate, up, down in each of the 16 layers
    (model.py:520-555) and the output head (model.py:560-565).  Each call here
    is that host-array call (x copied in, one launch, y copied out, the call
    returns when y is on the host), in the model's order over the synthetic
    1B model's own matrices, `tokens` times after one warm-up token.  The
    reference's own NumPy work between the calls (norms, RoPE, attention,
    SwiGLU) is not part of it."""
    import time

    import numpy as np

    from alpacca_amd.qmatrix import QuantMatrix
    mats = []
    for i in range(hp.n_layer):
        for name in DROP_IN_ORDER:
            t = tensors[f"blk.{i}.{name}.weight"]
            mats.append((name, QuantMatrix(t.data, t.dtype, t.shape[0], t.shape[1])))
    t = tensors["output.weight"]
    mats.append(("output", QuantMatrix(t.data, t.dtype, t.shape[0], t.shape[1])))
    xs = {m.cols: np.random.default_rng(m.cols).standard_normal(m.cols).astype(np.float32)
          for _, m in mats}
    per: dict = {}

    def token(record: bool):
        for name, m in mats:
            a = time.perf_counter()
            m.matvec(xs[m.cols])
            if record:
                per.setdefault((name, m.dtype), []).append(time.perf_counter() - a)

    token(False)
    a = time.perf_counter()
    for _ in range(tokens):
        token(True)
    ms = (time.perf_counter() - a) * 1e3 / tokens
    calls = {f"{n} {d}": {"calls_per_token": len(v) // tokens,
                          "us_median": round(float(np.median(v)) * 1e6, 1)}
             for (n, d), v in per.items()}
    n_calls = len(mats)
    log(f"drop-in host-array matvecs: {n_calls} calls per token, {ms:.2f} ms per token "
        f"({ms * 1e3 / n_calls:.1f} us per call)")
    del mats
    return {"calls_per_token": n_calls, "ms_per_token": round(ms, 3),
            "us_per_call_mean": round(ms * 1e3 / n_calls, 1), "per_matrix": calls,
            "tokens": tokens,
            "note": "QuantMatrix.matvec on NumPy arrays in model.py's call order (113 calls per "
                    "token), synchronous; the reference's NumPy work between the calls is not "
                    "included"}


def decode_ops() -> int:
    """Cost of each op type of the config-5 decode step inside a HIP graph:
    16 launches (one per layer, the model's own matrices and buffers) per
    measurement after a 2048-token prompt, HIP events around 5 replays."""
    import ctypes

    import numpy as np
    import torch

    from alpacca_amd import _lib
    from alpacca_amd.model import Model, synthetic_llama_1b
    from alpacca_amd.qmatrix import matvec_fused_device
    hp, tensors = synthetic_llama_1b(seed=0)
    m = Model(hp, tensors, n_ctx=DECODE_PROMPT + DECODE_GEN)
    del tensors
    prompt = [int(t) for t in np.random.default_rng(2048).integers(0, hp.n_vocab, DECODE_PROMPT)]
    m.generate_greedy(prompt, 4, graph=True)  # cache filled to ~2050 positions
    s, lib = m.stream, _lib.load()
    h = s.cuda_stream

    def ptr(t):
        return ctypes.c_void_p(t.data_ptr())

    def timed(fn, reps=5):
        with torch.cuda.stream(s):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for _ in range(reps):
                fn()
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            a.record(s)
            g.replay()
            b.record(s)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / reps

    st = ctypes.c_void_p(m.state.data_ptr())
    ops = {
        "q+k+v (RMSNorm fused, Q4_K+Q6_K one launch)": lambda: [
            m._matvecs([ly["attn_q"], ly["attn_k"], ly["attn_v"]], [m.q, m.k, m.v], m.x, h,
                       norm=ly["attn_norm"]) for ly in m.layers],
        "attention (rope, kv store, partials, combine)": lambda: [
            _lib.check(lib.aq_attention_rope(ptr(m.q), ptr(m.k), ptr(m.v), hp.n_head, hp.n_kv,
                                             hp.head_dim, hp.n_rot, 0, ptr(m.rope_cos),
                                             ptr(m.rope_sin), st, 0, m.n_ctx, ptr(m.kv[li, 0]),
                                             ptr(m.kv[li, 1]), ptr(m.att), ctypes.c_void_p(h)))
            for li in range(hp.n_layer)],
        "attn_output (accumulate)": lambda: [matvec_fused_device([ly["attn_output"]], m.att.data_ptr(),
                                                                 [m.o.data_ptr()], h, accumulate=True)
                                             for ly in m.layers],
        "gate+up (RMSNorm fused, SwiGLU in the store)": lambda: [
            matvec_fused_device([ly["ffn_gate_up"]], m.x.data_ptr(), [m.act.data_ptr()], h,
                                norm_w_ptr=ly["ffn_norm"].data_ptr(), eps=hp.rms_eps,
                                rmsnorm=True, swiglu_pairs=True) for ly in m.layers],
        "ffn_down (accumulate)": lambda: [
            matvec_fused_device([ly["ffn_down"]], m.act.data_ptr(), [m.o.data_ptr()], h,
                                accumulate=True) for ly in m.layers],
        "output head (RMSNorm fused), x16": lambda: [m._matvecs([m.output], [m.logits], m.x, h,
                                                                norm=m.out_norm) for _ in range(16)],
        "embedding row gather, x16": lambda: [m.tok_embd.rows_at_device(m.state.data_ptr(), 1,
                                                                        m.x.data_ptr(), h)
                                              for _ in range(16)],
    }
    out = {}
    for name, fn in ops.items():
        us = timed(fn) / 16
        out[name] = round(us, 2)
        log(f"{name:48s} {us:7.2f} us per launch group")

    def step():
        m._enqueue_layers()
        m._enqueue_head()
    out["layers + head (one step)"] = round(timed(step), 1)
    log(f"layers + head: {out['layers + head (one step)']} us")
    print(json.dumps({"decode_ops_us": out}), flush=True)
    return 0


def traffic_per_launch(algorithmic: int):
    """HBM bytes per dominant launch from the committed rocprofv3 counter runs
    (FETCH_SIZE + WRITE_SIZE of the same launches, each scaled by what the
    counter reads for a copy kernel of known size); None when absent, made
    for another launch size or for another kernel than the one timed."""
    try:
        t = json.loads(TRAFFIC_PROFILE.read_text())
    except (OSError, ValueError):
        return None
    if t.get("bytes_per_launch") != algorithmic or t.get("kernel_symbol") != DOMINANT:
        return None
    return t.get("hbm_bytes_per_launch")


def summarize(db: str, gate_up_launches: int, step_layers: int = 0) -> int:
    """Summary of a rocprofv3 results database of a run of this script:
    per-kernel duration statistics, then the last `gate_up_launches`
    dispatches of the dominant kernel (the roofline leg) with their counters
    when the run collected any, and the counters of the other kernels (the
    copies of a --calibrate run)."""
    import sqlite3

    import numpy as np
    con = sqlite3.connect(db)
    rows = con.execute("select dispatch_id, name, grid_x, workgroup_x, duration "
                       "from kernels order by start").fetchall()
    pmc: dict = {}
    try:
        for did, cname, val in con.execute(
                "select dispatch_id, counter_name, counter_value from pmc_events"):
            pmc.setdefault(did, {}).setdefault(cname, 0.0)
            pmc[did][cname] += val
    except sqlite3.Error:
        pass
    def short(name: str) -> str:  # the kernel and its template arguments
        name = name.replace("(anonymous namespace)::", "").replace("void ", "", 1)
        return name.split("(")[0].replace("aq::", "").replace(" ", "")[:70]

    by: dict = {}
    cnt: dict = {}
    for did, name, gx, wg, dur in rows:
        by.setdefault((short(name), gx, wg), []).append(dur / 1e3)
        for k, v in pmc.get(did, {}).items():
            cnt.setdefault((short(name), gx, wg), {}).setdefault(k, []).append(v)
    print(f"{'kernel':70s} {'grid':>8s} {'wg':>5s} {'calls':>6s} {'mean_us':>9s} "
          f"{'median_us':>9s} {'min_us':>8s}")
    for (name, gx, wg), d in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        d = np.array(d)
        extra = "".join(f"  {k} {np.mean(v):.1f}" for k, v in
                        sorted(cnt.get((name, gx, wg), {}).items()))
        print(f"{name:70s} {gx:8d} {wg:5d} {len(d):6d} {d.mean():9.3f} "
              f"{np.median(d):9.3f} {d.min():8.3f}{extra}")
    dom = [r for r in rows if DOMINANT in r[1]][-gate_up_launches:] if gate_up_launches else []
    if dom:
        d = np.array([r[4] for r in dom]) / 1e3
        print(f"\nroofline leg: last {len(dom)} dispatches of {DOMINANT}: mean {d.mean():.3f} us, "
              f"median {np.median(d):.3f} us, min {d.min():.3f} us, max {d.max():.3f} us")
        counters: dict = {}
        for r in dom:
            for k, v in pmc.get(r[0], {}).items():
                counters.setdefault(k, []).append(v)
        for k, v in sorted(counters.items()):
            print(f"  {k}: mean {np.mean(v):.1f} per dispatch")
    if step_layers:
        # the 8B step's graph: per layer q/k/v, attn_output, gate/up (the
        # single-step one-matrix kernel) and ffn_down (the several-step one),
        # in dispatch order; its replays are the leading run of that pattern
        # among the one-matrix dispatches (later legs break it)
        seq = [r for r in rows if short(r[1]).startswith("k_matvec_i8_one")]
        down = [("false" in short(r[1]).split(",")[3]) for r in seq]
        n = 0
        while n + 4 <= len(seq) and not any(down[n:n + 3]) and down[n + 3]:
            n += 4
        lay = seq[:n][-4 * step_layers:]
        names = ("q/k/v", "attn_output", "gate/up", "ffn_down")
        print(f"\n8B step launches by position (last {len(lay) // 4} layers of the step's "
              f"leading run of {n // 4} layers):")
        for i, nm in enumerate(names):
            d = np.array([r[4] for r in lay[i::4]]) / 1e3
            if len(d):
                print(f"  {nm:12s} mean {d.mean():6.2f} us  median {np.median(d):6.2f} us")
    for did, name, gx, wg, dur in rows:
        c = pmc.get(did, {})
        if c and "aq::" not in name:
            print(f"other kernel {short(name)} grid {gx}: {dur / 1e3:.2f} us, " +
                  ", ".join(f"{k} {v:.1f}" for k, v in sorted(c.items())))
    return 0


def calibrate() -> int:
    """Streaming ceiling: torch copy and sum of known sizes (rotating 4 buffers)."""
    import torch
    torch.cuda.init()
    dev = torch.device("cuda", 0)
    out: dict = {"calibration": []}
    for mb in (33, 128, 430):
        n = (mb << 20) // 4
        bufs = [torch.ones(n, dtype=torch.float32, device=dev) for _ in range(4)]
        dst = torch.empty(n, dtype=torch.float32, device=dev)
        for name, fn, moved in (("copy", lambda b: dst.copy_(b), 2), ("sum", lambda b: b.sum(), 1)):
            for b in bufs:
                fn(b)
            torch.cuda.synchronize()
            a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 5
            a.record()
            for _ in range(reps):
                for b in bufs:
                    fn(b)
            e.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(e) * 1e3 / (reps * len(bufs))
            gbs = moved * n * 4 / (us * 1e-6) / 1e9
            out["calibration"].append({"kernel": f"torch {name}", "bytes": n * 4,
                                       "bytes_moved": moved * n * 4,
                                       "us_per_launch": round(us, 2), "GB/s": round(gbs, 1)})
            log(f"{name} {mb} MB: {us:.2f} us/launch, {gbs:.0f} GB/s")
        del bufs, dst
    print(json.dumps(out), flush=True)
    return 0


def sizes() -> int:
    """Fixed and marginal cost of the gate/up launch: the int8 Q4_K kernel on
    2N x 4096 rows for N = 1024 .. 28672 (4.7 - 132 MB) as one matrix (the
    one-matrix launch the 8B step runs) and as two N x 4096 matrices in one
    multi-matrix launch, each size rotating over distinct copies (>= 700 MB,
    past the Infinity Cache) inside one HIP graph, and beside them the
    library's bare streaming read of the same rows (aq_stream_read, the
    better of 4096 and 8192 waves) and torch's sum over float buffers of the
    same byte counts.  A least-squares line through the sizes >= 9 MB gives
    each kernel's fixed cost per launch (graph dispatch included) and its
    marginal streaming rate."""
    import ctypes

    import numpy as np
    import torch

    from alpacca_amd import _lib, synth
    from alpacca_amd.qmatrix import QuantMatrix, matvec_multi_device
    dev = torch.device("cuda", 0)
    s = torch.cuda.Stream(dev)
    lib = _lib.ensure_device()
    sink = torch.zeros(4, dtype=torch.int32, device=dev)

    def timeit(fn, reps):
        with torch.cuda.stream(s):
            fn(0)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for r in range(reps):
                fn(r)
        best = float("inf")
        for _ in range(3):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(s):
                a.record(s)
                g.replay()
                b.record(s)
            torch.cuda.synchronize()
            best = min(best, a.elapsed_time(b) * 1e3 / reps)
        return best

    x = torch.from_numpy(synth.random_x(4096, seed=1)).to(dev)
    ys = [torch.empty(28672, device=dev) for _ in range(2)]
    raw = synth.random_matrix_bytes("Q4_K", 2 * 28672, 4096, seed=3)
    y1 = torch.empty(2 * 28672, device=dev)
    row_b = 2304
    rows = []
    for n in (1024, 2048, 4096, 7168, 14336, 28672):
        nb = 2 * n * row_b
        copies = max(4, int(700e6 // nb))
        mats = [QuantMatrix(raw[:2 * n * row_b], "Q4_K", 2 * n, 4096) for _ in range(copies)]
        one = timeit(lambda r: mats[r % copies].matvec_device(x.data_ptr(), y1.data_ptr(),
                                                              s.cuda_stream), 2 * copies)
        del mats
        mats = [(QuantMatrix(raw[:n * row_b], "Q4_K", n, 4096),
                 QuantMatrix(raw[n * row_b:2 * n * row_b], "Q4_K", n, 4096))
                for _ in range(copies)]
        us = timeit(lambda r: matvec_multi_device(list(mats[r % copies]), x.data_ptr(),
                                                  [ys[0].data_ptr(), ys[1].data_ptr()],
                                                  s.cuda_stream), 2 * copies)
        del mats
        bufs = [torch.ones(nb // 4, dtype=torch.float32, device=dev) for _ in range(copies)]
        rs = timeit(lambda r: bufs[r % copies].sum(), 2 * copies)
        # the bare streaming read of the same rows, best of two launch shapes
        rd = min(timeit(lambda r: _lib.check(lib.aq_stream_read(
            ctypes.c_void_p(bufs[r % copies].data_ptr()), 2 * n, row_b, waves, 1,
            ctypes.c_void_p(sink.data_ptr()), ctypes.c_void_p(s.cuda_stream))), 2 * copies)
            for waves in (4096, 8192))
        del bufs
        torch.cuda.empty_cache()
        rows.append({"rows": 2 * n, "bytes": nb, "one_matrix_us": round(one, 2),
                     "one_matrix_GBps": round(nb / one / 1e3, 1), "matvec_us": round(us, 2),
                     "matvec_GBps": round(nb / us / 1e3, 1), "read_us": round(rd, 2),
                     "read_GBps": round(nb / rd / 1e3, 1), "torch_sum_us": round(rs, 2),
                     "torch_sum_GBps": round(nb / rs / 1e3, 1)})
        log(f"gate/up 2x{n}x4096 ({nb / 1e6:.1f} MB): one matrix {one:.2f} us "
            f"({nb / one / 1e3:.0f} GB/s), two-matrix launch {us:.2f} us ({nb / us / 1e3:.0f} GB/s); "
            f"bare read {rd:.2f} us ({nb / rd / 1e3:.0f} GB/s); "
            f"torch sum {rs:.2f} us ({nb / rs / 1e3:.0f} GB/s)")
    mb = np.array([r["bytes"] for r in rows]) / 1e6
    fit = {}
    for key in ("one_matrix_us", "matvec_us", "read_us", "torch_sum_us"):
        t = np.array([r[key] for r in rows])
        big = mb >= 9
        c0, c1 = np.linalg.lstsq(np.vstack([np.ones(big.sum()), mb[big]]).T, t[big], rcond=None)[0]
        fit[key.replace("_us", "")] = {"fixed_us": round(float(c0), 2),
                                       "marginal_GBps": round(1e3 / float(c1), 1)}
    log(f"fit (>= 9 MB): {fit}")
    print(json.dumps({"sizes": rows, "fit": fit}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--separate", action="store_true",
                    help="one launch per projection instead of fused q/k/v and gate/up")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches")
    ap.add_argument("--steps-per-graph", type=int, default=0,
                    help="8B steps captured per HIP graph (replays of that graph while that "
                         "many steps remain, then one-step replays: exactly --steps steps); "
                         "0 = all --steps steps in one graph")
    ap.add_argument("--kernel", default="int8", choices=["int8", "fp32"])
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the config-5 synthetic 1B greedy decode")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the config-4 batched prefill (MFMA) timings")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the config 1-3 matvec shapes and the small-batch matmul_t leg")
    ap.add_argument("--configs-only", action="store_true",
                    help="run only the config 1-3 matvec leg (for counter runs)")
    ap.add_argument("--only", default="",
                    help="with --configs-only: shapes whose 'DTYPE ROWSxCOLS' contains this")
    ap.add_argument("--calibrate", action="store_true")
    ap.add_argument("--sizes", action="store_true",
                    help="fixed and marginal cost of the fused gate/up launch vs a read kernel")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the config-5 decode leg (for kernel traces of the step)")
    ap.add_argument("--small-batch-only", action="store_true",
                    help="run only the small-batch matmul_t leg (for counter runs)")
    ap.add_argument("--small-batch-formats", action="store_true",
                    help="run only the small-batch matmul_t of Q6_K and the per-32 formats")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the config-4 prefill leg (for counter runs)")
    ap.add_argument("--formats-only", action="store_true",
                    help="matmul_t at float32 accuracy for every exact-fp16 format (counter runs)")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="only the streaming-read ceiling at the gate/up launch's byte count")
    ap.add_argument("--decode-ops", action="store_true",
                    help="per-op cost of the config-5 decode step inside HIP graphs")
    ap.add_argument("--summarize", metavar="DB",
                    help="print the summary of a rocprofv3 results database of this script")
    ap.add_argument("--step-layers", type=int, default=0,
                    help="with --summarize: per-position launch times over the last N layers "
                         "of the 8B step's graph replays")
    ap.add_argument("--gate-up-launches", type=int, default=0,
                    help="with --summarize: dispatches of the roofline leg to single out "
                         "(its graph runs twice: 2 x layers x 12)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures a single GPU: --gpus {args.gpus} is not supported "
              "in this build (it measures one GPU's share of the hot path)", file=sys.stderr)
        return 2
    if args.summarize:
        return summarize(args.summarize, args.gate_up_launches, args.step_layers)
    if args.calibrate:
        return calibrate()
    if args.sizes:
        return sizes()
    if args.decode_ops:
        return decode_ops()
    if args.read_ceiling:
        import torch
        torch.cuda.init()
        dev = torch.device("cuda", 0)
        print(json.dumps({"read_ceiling": read_ceiling_leg(dev, torch.cuda.Stream(dev),
                                                           2 * q4k_bytes(14336, 4096))}),
              flush=True)
        return 0
    if args.configs_only:
        import torch
        torch.cuda.init()
        dev = torch.device("cuda", 0)
        global MATVEC_CONFIGS
        MATVEC_CONFIGS = [c for c in MATVEC_CONFIGS if args.only in f"{c[1]} {c[2]}x{c[3]}"]
        print(json.dumps({"matvec_configs": matvec_configs_leg(dev, torch.cuda.Stream(dev))}),
              flush=True)
        return 0
    if args.decode_only:
        from alpacca_amd.model import synthetic_llama_1b
        hp_1b, tensors_1b = synthetic_llama_1b(seed=0)
        print(json.dumps({"decode_1b": decode_leg(hp_1b, tensors_1b)}), flush=True)
        return 0
    if args.small_batch_only:
        import torch
        torch.cuda.init()
        dev = torch.device("cuda", 0)
        print(json.dumps({"small_batch": small_batch_leg(dev, torch.cuda.Stream(dev))}), flush=True)
        return 0
    if args.small_batch_formats:
        import torch
        torch.cuda.init()
        dev = torch.device("cuda", 0)
        print(json.dumps({"small_batch_formats": small_batch_formats_leg(
            dev, torch.cuda.Stream(dev))}), flush=True)
        return 0
    if args.prefill_only:
        import torch
        torch.cuda.init()
        dev = torch.device("cuda", 0)
        print(json.dumps({"prefill": prefill_leg(dev, torch.cuda.Stream(dev), reps=5)}), flush=True)
        return 0
    if args.formats_only:
        import torch
        torch.cuda.init()
        dev = torch.device("cuda", 0)
        print(json.dumps({"formats": prefill_leg(dev, torch.cuda.Stream(dev), reps=5,
                                                 cases=FORMAT_CASES)}), flush=True)
        return 0

    import numpy as np  # noqa: F401  (imported before torch, as elsewhere)
    import torch

    from alpacca_amd import synth
    from alpacca_amd.qmatrix import QuantMatrix, matvec_multi_device

    torch.cuda.init()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}; building {args.layers} layers")

    fused = not args.separate and args.kernel == "int8"
    # Fused: q/k/v uploaded as one 6144-row matrix and gate/up as one
    # 28672-row matrix (the same seeded bytes, rows concatenated; outputs
    # contiguous), as a loader fuses projections that share x, so each is a
    # one-matrix launch.  Separate: the seven matrices of each layer.
    groups = {"attn_qkv": ("attn_q", "attn_k", "attn_v"), "ffn_gate_up": ("ffn_gate", "ffn_up")}
    layers = []
    for layer in range(args.layers):
        mats, raw = {}, {}
        for si, (name, rows, cols) in enumerate(SHAPES_8B):
            raw[name] = (synth.random_matrix_bytes("Q4_K", rows, cols, seed=100 * layer + si),
                         rows, cols)
        if fused:
            for g, parts in groups.items():
                mats[g] = QuantMatrix(b"".join(bytes(raw[n][0]) for n in parts), "Q4_K",
                                      sum(raw[n][1] for n in parts), 4096)
            for name in ("attn_output", "ffn_down"):
                mats[name] = QuantMatrix(raw[name][0], "Q4_K", raw[name][1], raw[name][2])
            # the same projections as separate matrices (the Model's form)
            for g, parts in groups.items():
                for n in parts:
                    mats["sep_" + n] = QuantMatrix(raw[n][0], "Q4_K", raw[n][1], raw[n][2])
        else:
            for name, (data, rows, cols) in raw.items():
                mats[name] = QuantMatrix(data, "Q4_K", rows, cols)
        layers.append(mats)
    step_bytes = args.layers * sum(q4k_bytes(r, c) for _, r, c in SHAPES_8B)
    x4 = torch.from_numpy(synth.random_x(4096, seed=4096)).to(dev)
    x14 = torch.from_numpy(synth.random_x(14336, seed=14336)).to(dev)
    ys = {name: torch.empty(r, dtype=torch.float32, device=dev) for name, r, _ in SHAPES_8B}
    ys["attn_qkv"] = torch.empty(6144, dtype=torch.float32, device=dev)
    ys["ffn_gate_up"] = torch.empty(28672, dtype=torch.float32, device=dev)
    log(f"uploaded {sum(len(m) for m in layers)} matrices, {step_bytes / 1e6:.1f} MB per step")

    stream = torch.cuda.Stream(dev)  # default priority

    def gate_up(m, h: int) -> None:
        if fused:
            m["ffn_gate_up"].matvec_device(x4.data_ptr(), ys["ffn_gate_up"].data_ptr(), h)
        else:
            for name in ("ffn_gate", "ffn_up"):
                m[name].matvec_device(x4.data_ptr(), ys[name].data_ptr(), h, args.kernel)

    def step(h: int) -> None:
        for m in layers:
            if fused:
                m["attn_qkv"].matvec_device(x4.data_ptr(), ys["attn_qkv"].data_ptr(), h)
                m["attn_output"].matvec_device(x4.data_ptr(), ys["attn_output"].data_ptr(), h)
                gate_up(m, h)
                m["ffn_down"].matvec_device(x14.data_ptr(), ys["ffn_down"].data_ptr(), h)
            else:
                for name, _, cols in SHAPES_8B:
                    m[name].matvec_device((x14 if cols == 14336 else x4).data_ptr(),
                                          ys[name].data_ptr(), h, args.kernel)

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn(stream.cuda_stream)
        torch.cuda.synchronize()
        return g

    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            step(stream.cuda_stream)
    torch.cuda.synchronize()

    # K steps through HIP graphs of `per_graph` steps each, replayed while
    # that many steps remain, then one-step replays: exactly K steps, and a
    # graph replay's fixed cost (the runtime's, not the kernels') spread over
    # per_graph steps.  The product's decode loop replays graphs of several
    # steps the same way (Model.generate_greedy, steps_per_graph).
    def timed_steps(fn, per_graph: int) -> float:
        g1 = capture(fn)
        gk = None
        if per_graph > 1 and args.steps >= per_graph:
            def fk(h: int) -> None:
                for _ in range(per_graph):
                    fn(h)
            gk = capture(fk)
        with torch.cuda.stream(stream):
            for _ in range(args.warmup):
                g1.replay()
            if gk is not None:
                gk.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            a.record(stream)
            left = args.steps
            while gk is not None and left >= per_graph:
                gk.replay()
                left -= per_graph
            for _ in range(left):
                g1.replay()
            b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / args.steps

    # ---- timed region: K steps ----
    spg = args.steps if args.steps_per_graph <= 0 else args.steps_per_graph
    graph = not args.no_graph
    one_per_replay = None
    if graph:
        ms_per_step = timed_steps(step, spg)
        if spg > 1:  # the same steps at one graph replay per step, for comparison
            m1 = timed_steps(step, 1)
            one_per_replay = {"ms_per_step": round(m1, 5),
                              "GBps": round(step_bytes / (m1 * 1e-3) / 1e9, 1)}
            log(f"one step per graph replay: {m1:.4f} ms/step, {one_per_replay['GBps']:.1f} GB/s")
    else:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            start.record(stream)
            for _ in range(args.steps):
                step(stream.cuda_stream)
            end.record(stream)
        torch.cuda.synchronize()
        ms_per_step = start.elapsed_time(end) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"{args.steps} steps: {ms_per_step:.4f} ms/step, {value:.1f} GB/s")

    # ---- the same step in the decode step's own launch form: q/k/v and
    # gate/up as separate matrices, each group one multi-matrix launch
    # (matvec_multi, as Model runs them; the same bytes and launch count) ----
    multi = None
    if fused and graph:
        def step_multi(h: int) -> None:
            for m in layers:
                matvec_multi_device([m["sep_" + n] for n in groups["attn_qkv"]], x4.data_ptr(),
                                    [ys[n].data_ptr() for n in groups["attn_qkv"]], h)
                m["attn_output"].matvec_device(x4.data_ptr(), ys["attn_output"].data_ptr(), h)
                matvec_multi_device([m["sep_" + n] for n in groups["ffn_gate_up"]],
                                    x4.data_ptr(),
                                    [ys[n].data_ptr() for n in groups["ffn_gate_up"]], h)
                m["ffn_down"].matvec_device(x14.data_ptr(), ys["ffn_down"].data_ptr(), h)
        mms = timed_steps(step_multi, spg)
        multi = {"ms_per_step": round(mms, 5), "GBps": round(step_bytes / (mms * 1e-3) / 1e9, 1),
                 "hbm_fraction": round(step_bytes / (mms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                 "form": "q/k/v (3 matrices) and gate/up (2 matrices) as one multi-matrix launch "
                         "each, attn_output and ffn_down alone: the launch form of the decode "
                         "step (Model), same bytes, 4 launches per layer"}
        log(f"multi-matrix launch form: {mms:.4f} ms/step, {multi['GBps']:.1f} GB/s")

    # ---- roofline leg: the dominant launch (fused gate/up, one per layer),
    # ROOFLINE_REPS rounds over the layers captured as one graph ----
    per_layer = 1 if fused else 2

    def gate_up_rounds(h: int) -> None:
        for _ in range(ROOFLINE_REPS):
            for m in layers:
                gate_up(m, h)

    gu = capture(gate_up_rounds)
    with torch.cuda.stream(stream):
        for _ in range(2):
            gu.replay()
    torch.cuda.synchronize()
    # the average over ROOFLINE_REPLAYS replays (one replay's figure moved by
    # up to ~20 % between runs where the step and the read ceiling did not)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        a.record(stream)
        for _ in range(ROOFLINE_REPLAYS):
            gu.replay()
        b.record(stream)
    torch.cuda.synchronize()
    launches = ROOFLINE_REPLAYS * ROOFLINE_REPS * len(layers) * per_layer
    launch_us = a.elapsed_time(b) * 1e3 / launches
    kbytes = 2 * q4k_bytes(14336, 4096) // per_layer
    achieved = kbytes / (launch_us * 1e-6) / 1e9
    log(f"gate/up launches: {launches} in {a.elapsed_time(b):.3f} ms, {launch_us:.2f} us each "
        f"-> {achieved:.1f} GB/s")

    ceiling = read_ceiling_leg(dev, stream, kbytes)
    configs = None if args.no_configs else matvec_configs_leg(dev, stream)
    small = None if args.no_configs else small_batch_leg(dev, stream)
    prefill = None if args.no_prefill else prefill_leg(dev, stream)
    decode = None
    hp_1b = tensors_1b = None
    if not (args.no_decode and args.no_cpu):
        from alpacca_amd.model import synthetic_llama_1b
        hp_1b, tensors_1b = synthetic_llama_1b(seed=0)
    drop_in = None
    if not args.no_decode:
        decode = decode_leg(hp_1b, tensors_1b)
        drop_in = drop_in_leg(hp_1b, tensors_1b)

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline ({args.cpu_seconds:.0f} s budget)")
        cpu = cpu_baseline(args.cpu_seconds, tensors_1b, hp_1b)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} cores")
    del tensors_1b

    kernel_name = ("k_matvec_i8_one<UQ4K,1,3,true,512,0,false>: ffn_gate+ffn_up as one 28672x4096 "
                   "matrix, one launch"
                   if fused else f"{args.kernel} matvec: one ffn_gate or ffn_up launch, 14336x4096")
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
        "dtype": ("q4_k weights x f32 (int8x3-piece dot4, f32 combine)" if args.kernel == "int8"
                  else "f32"),
        "data": "synthetic: seeded GGUF Q4_K blocks (config 2 recipe), x ~ N(0,1) fp32",
        "config": {
            "workload": (f"Q4_K decode matvec (M=1) over {args.layers} distinct Llama-3-8B "
                         "layers x 7 projections (4096x4096, 1024x4096 x2, 4096x4096, "
                         "14336x4096 x2, 4096x14336); "
                         + ("q/k/v and gate/up each uploaded as one matrix, one launch each" if fused
                            else "one launch per projection")
                         + (f"; HIP graphs of {spg} steps (the timed steps in "
                            f"{args.steps // spg} replay(s) + {args.steps % spg} one-step "
                            "replay(s))" if graph else "; eager launches")),
            "steps_per_graph": spg if graph else None,
            "one_step_per_graph_replay": one_per_replay,
            "bytes_per_step": step_bytes,
            "hbm_fraction": round(value / HBM_PEAK_GBS, 4),
            "kernel": args.kernel,
            "other_legs": ("matvec_configs: configs 1-3 (C1 Q8_0 2048x2048; C2 Q4_K 2048x2048, "
                           "512x2048, 8192x2048, 2048x8192; C3 Q5_K 4096x4096, 1024x4096, "
                           "14336x4096, Q6_K 4096x14336 and 128256x4096), one M=1 launch each; "
                           "small_batch: matmul_t M=1/4/8/16/32/48 on Q4_K 14336x4096; prefill: config 4; "
                           "decode_1b: config 5; drop_in: the reference model.py's 113 "
                           "host-array matvec calls per token through QuantMatrix"),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_per_launch(kbytes) if fused else None,
            "kernel": kernel_name,
            "bytes_per_launch": kbytes, "us_per_launch": round(launch_us, 3),
            "launches_timed": launches,
            # the same byte count read by a bare streaming-read launch: what
            # one launch of this size can take from HBM on this part
            "read_ceiling": ceiling,
            "frac_of_read_ceiling": round(achieved / ceiling["GB/s"], 4),
        },
        "cpu_baseline": cpu,
        "step_multi_matrix_form": multi,
        "matvec_configs": configs,
        "small_batch": small,
        "prefill": prefill,
        "decode_1b": decode,
        "drop_in": drop_in,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
