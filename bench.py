#!/usr/bin/env python3
"""Benchmark of the MI355X GGUF quantized linear-layer path.

Headline: Q4_K GEMV (M=1) at K=4096 x N=14336, achieved HBM GB/s on the
packed-weight bytes.  A step is one GEMV launch over one full weight matrix.
Weights rotate over enough copies (>= 512 MiB) that the 256 MB Infinity Cache
cannot hold them, so every step streams its matrix from HBM.  Inputs are
resident in HBM before the timed region; launches are replayed from a captured
HIP graph on the launch stream, and HIP events on that stream bracket exactly
the timed launches.  GEMV weights carry their prepared mat-vec layout
(gollek_hip_weight_prepare, built once before timing, the same byte count);
the headline matrix is also timed on the GGUF bytes in place.

Secondary lines (in "extra"): the other GEMV configurations, the Q8_0 bf16
MFMA GEMM (M = 16 / 128 / 512; TFLOP/s at M = 512 is the metric's second
half) and the Q4_K MoE grouped FFN (hidden 2048 with the routed block, and
hidden 4096), each timed the same way; the GGUF file -> HBM upload rate
(gollek_hip_gguf_upload, wall clock).

cpu_baseline: the C restatement of the reference's Java raw mat-vec (oracle/)
on this host's cores, on the same Q4_K matrix (rank 0, N = 1 only).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--warm-seconds S] [--no-extra] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "Q4_K GEMV achieved HBM GB/s (% peak) @4096x14336; GEMM TFLOP/s M=512"
HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, published
BF16_PEAK_TFLOPS = 2500.0       # MI355X dense bf16 MFMA, published
ROTATION_BYTES = 640 * 2 ** 20  # > 512 MiB of distinct weight copies
PROFILE_DIR = REPO / "profiles"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=2000)
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument("--warm-seconds", type=float, default=1.0,
                   help="untimed GPU work before the first workload, so every timed run "
                        "sees the device at its steady-state clocks")
    p.add_argument("--no-extra", action="store_true")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--only", default="", help="comma list of workload names to run")
    p.add_argument("--eager", action="store_true",
                   help="launch each step directly instead of replaying a HIP graph")
    p.add_argument("--ceilings", action="store_true",
                   help="only measure the device's attainable figures: single-launch HBM read "
                        "time by size and grid (plain streaming kernels), the empty-launch "
                        "floor, and a hipBLASLt bf16 GEMM at M = 512 (one JSON line each)")
    p.add_argument("--ceiling-sizes", default="",
                   help="with --ceilings: comma list of byte sizes to sweep (default: all), "
                        "e.g. one size so a kernel trace maps each grid to its size")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a 256 MiB device-to-device copy 10 times (known HBM bytes, "
                        "used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


# ---- timing helpers ---------------------------------------------------------

class Rotation:
    """Device copies of one packed weight matrix, launched round robin."""

    def __init__(self, torch, host_bytes, type_id: int, rows: int, cols: int, prepared: bool = False,
                 copies: int = 0):
        from gollek_amd import tensor_ops as ops
        nbytes = host_bytes.size
        self.copies = copies or max(2, math.ceil(ROTATION_BYTES / nbytes))
        base = torch.from_numpy(host_bytes.reshape(-1)).cuda()
        self.buffers = [base] + [base.clone() for _ in range(self.copies - 1)]
        self.weights = [ops.DeviceWeight(type_id, b.data_ptr(), rows, cols) for b in self.buffers]
        if prepared:
            # Each copy's prepared mat-vec layout (gollek_hip_weight_prepare,
            # built once like a model-load step, outside any timed region; a
            # no-op for shapes without one): launches then stream the copy's
            # prepared bytes, as many as the GGUF bytes.
            for w in self.weights:
                w.prepare()
            torch.cuda.synchronize()
        self.nbytes = nbytes

    def close(self):
        for w in self.weights:
            w.close()


EAGER = False


def warm_device(torch, seconds: float) -> float:
    """Untimed fp32 matmuls for about `seconds`: the first timed launches of a
    cold process otherwise run below the device's steady-state clocks."""
    if seconds <= 0:
        return 0.0
    a = torch.randn(4096, 4096, device="cuda")
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            a = torch.mm(a, a).clamp_(-1.0, 1.0)
        torch.cuda.synchronize()
    return time.perf_counter() - t0


MIN_WARM_SECONDS = 0.05  # untimed replays of each workload before its timed region


def graph_time(torch, launch, copies: int, steps: int, warmup: int):
    """Times exactly `steps` launches; returns (ms per launch, launches timed).

    Launch i uses weight copy i % copies.  Untimed first: one eager pass over
    every copy, then replays of a graph of one full rotation until at least
    `warmup` launches and MIN_WARM_SECONDS have passed.  Timed: one replay of
    a graph of exactly `steps` launches starting at copy 0, so every copy is
    reused only after the others (>= 512 MiB) have been streamed, bracketed
    by HIP events on the launch stream.  With EAGER the timed launches are
    made directly on the stream instead of from a graph."""
    steps = max(1, int(steps))
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for i in range(copies):  # eager warm-up before capture
            launch(i, stream.cuda_stream)
    stream.synchronize()
    warm = torch.cuda.CUDAGraph()
    with torch.cuda.graph(warm, stream=stream):
        s = torch.cuda.current_stream().cuda_stream
        for i in range(copies):
            launch(i, s)
    done, t0 = 0, time.perf_counter()
    with torch.cuda.stream(stream):
        while done < warmup or time.perf_counter() - t0 < MIN_WARM_SECONDS:
            warm.replay()
            stream.synchronize()
            done += copies
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    if EAGER:
        with torch.cuda.stream(stream):
            start.record(stream)
            for i in range(steps):
                launch(i % copies, stream.cuda_stream)
            end.record(stream)
    else:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            s = torch.cuda.current_stream().cuda_stream
            for i in range(steps):
                launch(i % copies, s)
        with torch.cuda.stream(stream):
            start.record(stream)
            g.replay()
            end.record(stream)
    end.synchronize()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, steps


# ---- workloads ----------------------------------------------------------------

def gemv_workload(torch, type_id: int, rows: int, cols: int, steps: int, warmup: int, seed: int,
                  prepared: bool = True, copies: int = 0):
    from gollek_amd import synthetic as syn
    host = syn.matrix(type_id, rows, cols, seed)
    rot = Rotation(torch, host, type_id, rows, cols, prepared, copies)
    x = torch.from_numpy(syn.activation(cols, seed + 1)).cuda()
    y = torch.empty(rows, dtype=torch.float32, device="cuda")

    def launch(i, stream):
        rot.weights[i].matvec(x.data_ptr(), y.data_ptr(), rows, stream)

    ms, n = graph_time(torch, launch, rot.copies, steps, warmup)
    algo_bytes = rot.nbytes + 4 * cols + 4 * rows
    res = {
        "ms_per_step": ms, "steps": n, "weight_copies": rot.copies, "prepared_layout": prepared,
        "weight_bytes": int(rot.nbytes), "algo_bytes": int(algo_bytes),
        "weight_gbs": rot.nbytes / (ms * 1e-3) / 1e9,
        "algo_gbs": algo_bytes / (ms * 1e-3) / 1e9,
        "gflops": 2.0 * rows * cols / (ms * 1e-3) / 1e9,
    }
    rot.close()
    return res, host


def gemm_workload(torch, m: int, steps: int, warmup: int, seed: int, type_id: int = 8,
                  rows: int = 4096, cols: int = 4096):
    from gollek_amd import synthetic as syn
    host = syn.matrix(type_id, rows, cols, seed)
    rot = Rotation(torch, host, type_id, rows, cols)
    xb = torch.from_numpy(syn.activation_bf16(m, cols, seed + 1).view("int16")).cuda()
    y = torch.empty((m, rows), dtype=torch.float32, device="cuda")

    def launch(i, stream):
        rot.weights[i].gemm_bf16(xb.data_ptr(), m, y.data_ptr(), stream)

    ms, n = graph_time(torch, launch, rot.copies, steps, warmup)
    flops = 2.0 * m * rows * cols
    algo_bytes = rot.nbytes + 2 * m * cols + 4 * m * rows
    res = {
        "ms_per_step": ms, "steps": n, "m": m, "weight_copies": rot.copies,
        "tflops": flops / (ms * 1e-3) / 1e12,
        "mfma_frac": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
        "algo_gbs": algo_bytes / (ms * 1e-3) / 1e9,
    }
    rot.close()
    return res, host


def moe_workload(torch, steps: int, warmup: int, seed: int, shape=(128, 8, 2048, 768, 16),
                 copies: int = 3, routed: bool = True, types=None, global_experts: int = 0):
    """Grouped expert FFN, shape (experts, top_k, hidden, inter, tokens),
    expert types (gate, up, down) (default Q4_K); with `routed`, also the
    routed block (router -> top-k -> the same FFN).  Weights rotate over
    `copies` whole layers.  global_experts > experts: one GPU's share of an
    expert-parallel layer -- the routes are drawn over the global experts
    and those outside this GPU's (the first `experts`) carry id -1, which
    the grouped FFN skips."""
    import numpy as np

    from gollek_amd import synthetic as syn
    from gollek_amd import tensor_ops as ops
    E, k, H, I, T = shape
    tg, tu, td = types or (syn.Q4_K, syn.Q4_K, syn.Q4_K)
    gate = syn.matrix(tg, E * I, H, seed)
    up = syn.matrix(tu, E * I, H, seed + 1)
    down = syn.matrix(td, E * H, I, seed + 2)
    ids, w = syn.moe_routing(T, global_experts or E, k, seed + 3)
    ids = np.where(ids < E, ids, -1).astype(np.int32)
    x = syn.activation(T * H, seed + 4).reshape(T, H)
    # At 128 x 2048 x 768, three copies of the whole layer (3 x 340 MB): a copy
    # is reused only after the other two layers' touched experts (> 400 MB)
    # have streamed, so the 256 MB Infinity Cache cannot serve it.
    layers = []
    for _ in range(copies):
        bufs = [torch.from_numpy(a.reshape(-1)).cuda() for a in (gate, up, down)]
        handles = (ops.DeviceWeight(tg, bufs[0].data_ptr(), E * I, H),
                   ops.DeviceWeight(tu, bufs[1].data_ptr(), E * I, H),
                   ops.DeviceWeight(td, bufs[2].data_ptr(), E * H, I))
        layers.append((bufs, handles))
    ws_bytes = ops.moe_workspace_bytes(T, k, H, I, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    xd = torch.from_numpy(x).cuda()
    idd = torch.from_numpy(ids).cuda()
    wd = torch.from_numpy(w).cuda()
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")

    def launch(i, stream):
        g, u, d = layers[i][1]
        ops.moe_grouped_device(g, u, d, E, xd.data_ptr(), idd.data_ptr(), wd.data_ptr(), T, k,
                               out.data_ptr(), ws.data_ptr(), ws_bytes, stream)

    ms, n = graph_time(torch, launch, copies, steps, warmup)
    used = len(np.unique(ids[ids >= 0]))
    bytes_used = used * (gate.size // E + up.size // E + down.size // E) + 2 * T * H * 4
    res = {"ms_per_step": ms, "steps": n, "experts_touched": int(used),
           "algo_bytes": int(bytes_used), "algo_gbs": bytes_used / (ms * 1e-3) / 1e9,
           "hbm_frac": bytes_used / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "shape": {"experts": E, "top_k": k, "hidden": H, "inter": I, "tokens": T},
           "routes": int((ids >= 0).sum())}
    if global_experts:
        res["shape"]["global_experts"] = global_experts
    if not routed:
        for _, handles in layers:
            for h in handles:
                h.close()
        return res, (gate, up, down, E, H, I, x, ids, w)

    # The routed block: router logits (seeded N(0, 2^2)) -> sigmoid top-8 on the
    # GPU -> the same grouped FFN (gollek_hip_moe_block_device).
    logits = torch.from_numpy(
        (2.0 * np.random.default_rng(seed + 5).standard_normal((T, E))).astype(np.float32)).cuda()
    bids = torch.empty((T, k), dtype=torch.int32, device="cuda")
    bw = torch.empty((T, k), dtype=torch.float32, device="cuda")

    def launch_block(i, stream):
        g, u, d = layers[i][1]
        ops.moe_block_device(g, u, d, E, xd.data_ptr(), logits.data_ptr(), T, k,
                             ops.ROUTER_SIGMOID, bids.data_ptr(), bw.data_ptr(), out.data_ptr(),
                             ws.data_ptr(), ws_bytes, stream)

    bms, bn = graph_time(torch, launch_block, copies, steps, warmup)
    bused = len(np.unique(bids.cpu().numpy()))
    bbytes = bused * (gate.size // E + up.size // E + down.size // E) + 2 * T * H * 4 \
        + T * E * 4
    res["routed_block"] = {"ms_per_step": bms, "steps": bn, "experts_touched": int(bused),
                           "scoring": "sigmoid", "algo_bytes": int(bbytes),
                           "algo_gbs": bbytes / (bms * 1e-3) / 1e9}
    for _, handles in layers:
        for h in handles:
            h.close()
    return res, (gate, up, down, E, H, I, x, ids, w)


def host_entry_workload(host, rows: int, cols: int, steps: int, warmup: int):
    """The host-buffer entry point (gollek_hip_matvec_rows): x copied in, y
    copied back and the stream synchronized on every call, as the Java seam
    calls it.  Weights are device-resident handles, rotated like the device
    workloads.  PCIe- and call-overhead inclusive; reported, never `value`."""
    import numpy as np

    from gollek_amd import synthetic as syn
    from gollek_amd import tensor_ops as ops
    copies = max(2, math.ceil(ROTATION_BYTES / host.size))
    tensors = [ops.GgufTensor(f"blk.{i}.ffn_up.weight", (cols, rows), syn.Q4_K, host)
               for i in range(copies)]
    for t in tensors:
        t.handle()
    x = syn.activation(cols, 3)
    y = np.empty(rows, dtype=np.float32)
    for i in range(max(warmup, copies)):
        ops.mat_vec_rows(tensors[i % copies], x, y, rows)
    n = max(steps, copies)
    t0 = time.perf_counter()
    for i in range(n):
        ops.mat_vec_rows(tensors[i % copies], x, y, rows)
    dt = (time.perf_counter() - t0) / n
    for t in tensors:
        t.close()
    return {"us_per_call": dt * 1e6, "calls": n, "weight_gbs": host.size / dt / 1e9,
            "note": "host float[] in/out per call (PCIe + sync inclusive); weights resident"}


def gguf_upload_workload(host, rows: int, cols: int, copies: int = 8):
    """GGUF file -> device handles (gollek_hip_gguf_upload): a file holding
    `copies` Q4_K rows x cols tensors is written to a temporary directory,
    opened with the native loader and every tensor uploaded.  The file was
    just written, so its pages are in the host page cache: this is the
    mapped-file -> pinned staging -> HBM rate, not a disk rate.  The first
    upload (which also allocates the pinned staging buffers) is untimed."""
    import shutil
    import tempfile

    from gollek_amd import _native
    from gollek_amd import tensor_ops as ops
    from gollek_amd import gguf_writer as gw

    blobs = [(f"blk.{i}.ffn_up.weight", (cols, rows), 12, host.tobytes()) for i in range(copies + 1)]
    tmp = tempfile.mkdtemp(prefix="gguf_bench_")
    try:
        path = os.path.join(tmp, "model.gguf")
        with open(path, "wb") as fh:
            fh.write(gw.gguf_file([("general.alignment", gw.U32, 32)], blobs)[0])
        lib = _native.load()
        with ops.GgufFile(path) as f:
            lib.gollek_hip_weight_free(f.upload(0))
            t0 = time.perf_counter()
            handles = [f.upload(i) for i in range(1, copies + 1)]
            dt = time.perf_counter() - t0
            for h in handles:
                lib.gollek_hip_weight_free(h)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    nbytes = host.size * copies
    return {"tensors": copies, "bytes": nbytes, "ms_per_tensor": dt / copies * 1e3,
            "upload_gbs": nbytes / dt / 1e9,
            "note": "page-cache-resident GGUF file -> pinned staging -> HBM (synchronous per tensor)"}


# ---- CPU baseline -------------------------------------------------------------

def _cpu_median(fn, min_reps: int = 10, budget_s: float = 3.0, max_reps: int = 200):
    """Median seconds of fn() over >= min_reps runs after 2 warm-ups (more
    runs while the budget lasts); returns (median, runs)."""
    for _ in range(2):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_gemv(type_id: int, host, cols: int, label: str, budget_s: float = 3.0):
    """The oracle (C restatement of the reference's Java raw mat-vec route,
    scheduled like RT/GgufParallelConfig: all host cores, 2T row chunks) over
    the whole matrix, plus a single-thread rate on its first 1024 rows."""
    from gollek_amd import synthetic as syn
    from oracle import oracle as o
    x = syn.activation(cols, 99)
    threads = o.default_threads()
    med, n = _cpu_median(lambda: o.matvec(type_id, host, cols, x, threads=threads), budget_s=budget_s)
    sub = host[:1024]
    st, _ = _cpu_median(lambda: o.matvec(type_id, sub, cols, x, threads=1), min_reps=5, budget_s=1.0,
                        max_reps=20)
    return {
        "value": host.size / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"full {label} matrix ({host.size} packed bytes), median of {n} reps after 2 "
                   f"warm-ups, {threads} threads; C restatement of the reference Java raw route "
                   f"(oracle/gguf_oracle.c)"),
        "ms_per_matvec": med * 1e3,
        "single_thread_gbs": sub.size / st / 1e9,
    }


def cpu_baseline(host, cols: int):
    """cpu_baseline of the headline Q4_K 14336 x 4096 matrix."""
    from gollek_amd import synthetic as syn
    return cpu_gemv(syn.Q4_K, host, cols, "Q4_K 14336x4096", budget_s=5.0)


def cpu_gemm(host, m: int, seed: int, type_id: int = 8, cols: int = 4096):
    """The reference's prefill for one Linear: m independent matVecRows
    (RT/GgufTensorOps.java:666-674) over the rows of X (bf16 -> fp32
    exactly), each on all host cores.  Bounded: >= 3 reps."""
    from gollek_amd import synthetic as syn
    from oracle import oracle as o
    xb = syn.activation_bf16(m, cols, seed)
    x = syn.bf16_to_f32(xb).reshape(m, cols)
    threads = o.default_threads()

    def run():
        for r in range(m):
            o.matvec(type_id, host, cols, x[r], threads=threads)

    med, n = _cpu_median(run, min_reps=3, budget_s=2.0, max_reps=50)
    flops = 2.0 * m * host.shape[0] * cols
    return {"value": flops / med / 1e9, "unit": "GFLOP/s", "cores": threads, "kind": "port",
            "ms_per_gemm": med * 1e3, "weight_gbs_per_row_pass": host.size * m / med / 1e9,
            "sample": (f"{m} mat-vecs of the {host.shape[0]}x{cols} matrix (one per row of X), median "
                       f"of {n} reps after 2 warm-ups, {threads} threads per mat-vec; oracle")}


def cpu_moe(gate, up, down, E: int, H: int, I: int, x, ids, wts):
    """The reference's MoE expert loop (MoeForwardPass.java:217-240 with
    swigluFfn): per token and route, gate and up mat-vecs of the expert's
    Q4_K rows, silu(g) * u in fp32, the down mat-vec and the weighted add,
    each mat-vec on all host cores (oracle)."""
    import numpy as np

    from gollek_amd import synthetic as syn
    from oracle import oracle as o
    threads = o.default_threads()
    T, k = ids.shape

    def run():
        out = np.zeros((T, H), np.float32)
        for t in range(T):
            for j in range(k):
                e, wj = int(ids[t, j]), np.float32(wts[t, j])
                g = o.matvec(syn.Q4_K, gate[e * I:(e + 1) * I], H, x[t], threads=threads)
                u = o.matvec(syn.Q4_K, up[e * I:(e + 1) * I], H, x[t], threads=threads)
                with np.errstate(over="ignore"):  # exp(-g) = inf: silu -> -0
                    h = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
                out[t] += wj * o.matvec(syn.Q4_K, down[e * H:(e + 1) * H], I, h, threads=threads)
        return out

    med, n = _cpu_median(run, min_reps=5, budget_s=3.0, max_reps=50)
    pair_bytes = gate.shape[1] * I * 2 + down.shape[1] * H
    return {"value": T * k * pair_bytes / med / 1e9, "unit": "GB/s (weights streamed per route)",
            "cores": threads, "kind": "port", "ms_per_layer": med * 1e3,
            "sample": (f"{T} tokens x top-{k} of {E} Q4_K experts (H {H}, I {I}), every route's "
                       f"expert read per route as the reference does; median of {n} reps after 2 "
                       f"warm-ups, {threads} threads per mat-vec; oracle")}


def ceilings(torch, steps: int, warmup: int, only_sizes=()) -> int:
    """Attainable HBM read time per launch (libgollek_ceiling.so: plain
    streaming reads, every load issued up front) by size, load kind and grid;
    the empty-launch floor; a hipBLASLt bf16 GEMM (torch.nn.functional.linear)
    at M = 512, K = N = 4096 on pre-dequantized weights.  Timed exactly like
    the workloads (graph_time over a >= 640 MiB rotation)."""
    import ctypes

    lib = ctypes.CDLL(str(REPO / "gollek_amd" / "libgollek_ceiling.so"))
    lib.gollek_ceiling_loads_per_lane.restype = ctypes.c_int64
    lib.gollek_ceiling_loads_per_lane.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                                  ctypes.c_int32]
    lib.gollek_ceiling_launch.restype = ctypes.c_int32
    lib.gollek_ceiling_launch.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_int64,
                                          ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.c_void_p]
    kinds = {0: "reg_nt", 1: "reg", 2: "lds_nt", 3: "empty"}
    out = torch.empty(16384 * 1024, dtype=torch.int32, device="cuda")
    best = {}

    def run(kind, nbytes, bufs, blocks, wpb):
        if lib.gollek_ceiling_loads_per_lane(kind, nbytes, blocks, wpb) < 0:
            return
        ptrs = [b.data_ptr() for b in bufs]
        if lib.gollek_ceiling_launch(kind, ptrs[0], nbytes, out.data_ptr(), blocks, wpb, None) != 0:
            return
        torch.cuda.synchronize()

        def launch(i, st):
            lib.gollek_ceiling_launch(kind, ptrs[i], nbytes, out.data_ptr(), blocks, wpb, st)

        ms, n = graph_time(torch, launch, len(ptrs), steps, warmup)
        rec = {"ceiling": "hbm_read", "kind": kinds[kind], "bytes": nbytes, "blocks": blocks,
               "waves_per_block": wpb, "us": round(ms * 1e3, 3), "steps": n,
               "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1) if nbytes else None}
        print(json.dumps(rec), flush=True)
        key = (kinds[kind] if kind == 3 else "read", nbytes)
        if key not in best or rec["us"] < best[key]["us"]:
            best[key] = rec

    sizes = (33030144, 2 * 2 ** 20, 8 * 2 ** 20, 17825792, 25362432, 64 * 2 ** 20,
             128 * 2 ** 20, 295501824)
    if only_sizes:
        sizes = tuple(only_sizes)
    for nbytes in sizes:
        copies = max(2, math.ceil(ROTATION_BYTES / nbytes))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
        for b in bufs:
            b.fill_(0x5A)
        kset = (0, 1, 2) if nbytes == 33030144 else (0, 2)
        for kind in kset:
            for wpb in (4, 8, 16):
                for blocks in (256, 512, 768, 1024, 2048, 4096, 8192):
                    run(kind, nbytes, bufs, blocks, wpb)
        del bufs
    for blocks in (256, 896, 1024, 4096):
        run(3, 0, [out], blocks, 4)
    # hipBLASLt bf16 GEMM, Y = X W^T, M = 512, K = N = 4096
    M = K = N = 4096
    M = 512
    wbytes = 2 * N * K
    copies = max(2, math.ceil(ROTATION_BYTES / wbytes))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    ws = [torch.randn(N, K, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(copies)]
    xb = torch.randn(M, K, device="cuda", generator=gen).to(torch.bfloat16)
    yb = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)

    def gemm(i, st):
        torch.nn.functional.linear(xb, ws[i], out=yb)

    ms, n = graph_time(torch, gemm, copies, steps, warmup)
    rec = {"ceiling": "bf16_gemm_hipblaslt", "m": M, "n": N, "k": K, "us": round(ms * 1e3, 3),
           "steps": n, "tflops": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1),
           "op": "torch.nn.functional.linear(bf16 X, bf16 W) -> bf16 Y"}
    print(json.dumps(rec), flush=True)
    summary = {"ceiling_summary": [best[k] for k in sorted(best, key=lambda k: (k[0], k[1]))],
               "bf16_gemm_m512_tflops": rec["tflops"]}
    print(json.dumps(summary), flush=True)
    return 0


def traffic_from_profile():
    """HBM bytes per launch of the headline kernel from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel
    calibration recorded in the same file), or None."""
    path = PROFILE_DIR / "q4k_gemv_4096x14336_pmc.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get("hbm_bytes_per_launch")
    except Exception:
        return None


def main() -> int:
    args = parse()
    global EAGER
    EAGER = args.eager
    if args.copy_calibration:
        import torch
        n = 256 * 2 ** 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n, "copy_calibration_bytes_written": n,
                          "copies": 10}))
        return 0
    if args.ceilings:
        import torch
        return ceilings(torch, min(args.steps, 400), args.warmup,
                        [int(v) for v in args.ceiling_sizes.split(",") if v])
    if args.gpus != 1:
        print(json.dumps({"error": "single-GPU build: this path runs on one GPU; "
                                   f"--gpus {args.gpus} is not supported (use --gpus 1)"}))
        log(f"--gpus {args.gpus} requested: only the one-GPU path exists; exiting")
        return 2
    import torch
    from gollek_amd import synthetic as syn
    from gollek_amd import tensor_ops as ops

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    ops.init(0)
    only = set(filter(None, args.only.split(",")))

    def want(name):
        return not only or name in only

    warmed = warm_device(torch, args.warm_seconds)
    log(f"device warm-up {warmed:.2f} s")
    log("headline: Q4_K GEMV K=4096 N=14336")
    head, host = gemv_workload(torch, syn.Q4_K, 14336, 4096, args.steps, args.warmup, seed=2)
    log(f"headline {head['weight_gbs']:.1f} GB/s, {head['ms_per_step'] * 1e3:.2f} us/launch")

    extra = {}
    hosts = {}  # workload -> host copy of its weights (for the CPU baselines)
    moe_inputs = gemm_host = None
    if not args.no_extra:
        for name, t, rows, cols in (("q8_0_gemv_4096x4096", syn.Q8_0, 4096, 4096),
                                    ("q4_0_gemv_4096x11008", syn.Q4_0, 11008, 4096),
                                    ("q4_k_gemv_4096x128256", syn.Q4_K, 128256, 4096),
                                    ("q6_k_gemv_14336x4096", syn.Q6_K, 4096, 14336),
                                    ("q6_k_gemv_4096x128256", syn.Q6_K, 128256, 4096),
                                    ("q5_k_gemv_4096x4096", syn.Q5_K, 4096, 4096),
                                    ("q5_k_gemv_14336x4096", syn.Q5_K, 4096, 14336),
                                    ("q4_k_gemv_14336x4096", syn.Q4_K, 4096, 14336),
                                    ("q4_0_gemv_11008x4096", syn.Q4_0, 4096, 11008)):
            if not want(name):
                continue
            log(f"extra {name}")
            r, hosts[name] = gemv_workload(torch, t, rows, cols, args.steps, args.warmup, seed=5)
            r["hbm_frac"] = r["weight_gbs"] / HBM_PEAK_GBS
            extra[name] = r
        if want("q4_k_gemv_4096x14336_gguf_layout"):
            # The headline matrix without its prepared layout: the column
            # kernel reading the GGUF rows in place.
            log("extra headline on the GGUF layout")
            r, _ = gemv_workload(torch, syn.Q4_K, 14336, 4096, args.steps, args.warmup, seed=2, prepared=False)
            r["hbm_frac"] = r["weight_gbs"] / HBM_PEAK_GBS
            extra["q4_k_gemv_4096x14336_gguf_layout"] = r
        # One GPU's share of a sharded layer: the headline matrix at 8-way
        # tensor parallelism (1792 of its 14336 rows, 4.13 MB) streamed from
        # HBM over a rotation of copies and, as a sharded layer would run it,
        # resident in the Infinity Cache (two copies); and one of 8
        # expert-parallel GPUs of the MoE layer (16 of 128 experts, only the
        # routes to them).
        if want("q4_k_gemv_4096x1792_tp8_share"):
            log("extra q4_k_gemv_4096x1792_tp8_share")
            r, _ = gemv_workload(torch, syn.Q4_K, 1792, 4096, args.steps, args.warmup, seed=2)
            r["hbm_frac"] = r["weight_gbs"] / HBM_PEAK_GBS
            r["mall_resident"], _ = gemv_workload(torch, syn.Q4_K, 1792, 4096, args.steps, args.warmup,
                                                  seed=2, copies=2)
            extra["q4_k_gemv_4096x1792_tp8_share"] = r
        if _has_symbol("gollek_hip_moe_grouped_device") and want("moe_q4_k_e16_of_128_ep8_share"):
            log("extra moe_q4_k_e16_of_128_ep8_share")
            extra["moe_q4_k_e16_of_128_ep8_share"], _ = moe_workload(
                torch, args.steps, args.warmup, seed=11, shape=(16, 8, 2048, 768, 16), copies=24,
                routed=False, global_experts=128)
        have_gemm = hasattr(ops.DeviceWeight, "gemm_bf16") and _has_symbol("gollek_hip_gemm_bf16_device")
        for m in (16, 128, 512):
            name = f"q8_0_gemm_bf16_m{m}_4096x4096"
            if have_gemm and want(name):
                log(f"extra {name}")
                extra[name], gemm_host = gemm_workload(torch, m, args.steps, args.warmup, seed=7)
        # Q4_K / Q4_0 / Q5_K / Q6_K weights at the FFN shape (K 4096, N 14336).
        for tname, t, ms in (("q4_k", syn.Q4_K, (2, 4, 16, 128, 512)), ("q4_0", syn.Q4_0, (128, 512)),
                             ("q5_k", syn.Q5_K, (16, 128, 512)), ("q6_k", syn.Q6_K, (16, 128, 512))):
            for m in ms:
                name = f"{tname}_gemm_bf16_m{m}_4096x14336"
                if have_gemm and want(name):
                    log(f"extra {name}")
                    extra[name], hosts[name] = gemm_workload(torch, m, args.steps, args.warmup, seed=9,
                                                             type_id=t, rows=14336, cols=4096)
        # Batched decode through the FFN down projection (K 14336, N 4096).
        name = "q4_k_gemm_bf16_m2_14336x4096"
        if have_gemm and want(name):
            log(f"extra {name}")
            extra[name], hosts[name] = gemm_workload(torch, 2, args.steps, args.warmup, seed=9,
                                                     type_id=syn.Q4_K, rows=4096, cols=14336)
        if want("q4_k_gemv_host_entry_4096x14336"):
            log("extra host-buffer entry point")
            extra["q4_k_gemv_host_entry_4096x14336"] = host_entry_workload(
                host, 14336, 4096, args.steps, args.warmup)
        if _has_symbol("gollek_hip_moe_grouped_device") and want("moe_q4_k_e128_top8_t16"):
            log("extra moe")
            extra["moe_q4_k_e128_top8_t16"], moe_inputs = moe_workload(torch, args.steps, args.warmup,
                                                                      seed=11)
        # Batched decode and prefill: 64, 256 and 512 tokens through the same
        # layer (every expert takes several to tens of routes).
        for T in (64, 256, 512):
            name = f"moe_q4_k_e128_top8_t{T}"
            if _has_symbol("gollek_hip_moe_grouped_device") and want(name):
                log(f"extra {name}")
                extra[name] = moe_workload(torch, args.steps, args.warmup, seed=17,
                                           shape=(128, 8, 2048, 768, T), routed=False)[0]
        if _has_symbol("gollek_hip_moe_grouped_device") and want("moe_q4_k_e128_top8_t16_h4096"):
            log("extra moe hidden 4096")
            # 128 experts, top-8, hidden 4096, inter 1536 (two 1.36 GB layers
            # of which 860 MB are touched: past the Infinity Cache)
            extra["moe_q4_k_e128_top8_t16_h4096"] = moe_workload(
                torch, args.steps, args.warmup, seed=13, shape=(128, 8, 4096, 1536, 16), copies=2,
                routed=False)[0]
        # Other expert types at the same shape: Q4_K or Q5_K gate / up with
        # Q6_K down (Q4_K_M / Q5_K_M files' layers), all-Q5_K (Q5_K_S), all-Q6_K,
        # all-Q8_0 and all-Q4_0.
        for name, types in (("moe_q4_k_q6_k_down_e128_top8_t16", (syn.Q4_K, syn.Q4_K, syn.Q6_K)),
                            ("moe_q5_k_q6_k_down_e128_top8_t16", (syn.Q5_K, syn.Q5_K, syn.Q6_K)),
                            ("moe_q5_k_e128_top8_t16", (syn.Q5_K, syn.Q5_K, syn.Q5_K)),
                            ("moe_q6_k_e128_top8_t16", (syn.Q6_K, syn.Q6_K, syn.Q6_K)),
                            ("moe_q8_0_e128_top8_t16", (syn.Q8_0, syn.Q8_0, syn.Q8_0)),
                            ("moe_q4_0_e128_top8_t16", (syn.Q4_0, syn.Q4_0, syn.Q4_0))):
            if _has_symbol("gollek_hip_moe_grouped_device") and want(name):
                log(f"extra {name}")
                extra[name] = moe_workload(torch, args.steps, args.warmup, seed=11, routed=False,
                                           types=types)[0]
        if _has_symbol("gollek_hip_gguf_upload") and want("gguf_upload_q4_k_4096x14336"):
            log("extra gguf upload")
            extra["gguf_upload_q4_k_4096x14336"] = gguf_upload_workload(host, 14336, 4096)

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle restatement of the reference raw route)")
        cpu = cpu_baseline(host, 4096)
        # The other configurations, each on a bounded sample (a few seconds).
        cpus = {}
        for name, t, cols, label in (("q8_0_gemv_4096x4096", syn.Q8_0, 4096, "Q8_0 4096x4096"),
                                     ("q4_0_gemv_4096x11008", syn.Q4_0, 4096, "Q4_0 11008x4096"),
                                     ("q4_k_gemv_4096x128256", syn.Q4_K, 4096, "Q4_K 128256x4096"),
                                     ("q6_k_gemv_14336x4096", syn.Q6_K, 14336, "Q6_K 4096x14336"),
                                     ("q6_k_gemv_4096x128256", syn.Q6_K, 4096, "Q6_K 128256x4096"),
                                     ("q5_k_gemv_4096x4096", syn.Q5_K, 4096, "Q5_K 4096x4096"),
                                     ("q5_k_gemv_14336x4096", syn.Q5_K, 14336, "Q5_K 4096x14336"),
                                     ("q4_k_gemv_14336x4096", syn.Q4_K, 14336, "Q4_K 4096x14336"),
                                     ("q4_0_gemv_11008x4096", syn.Q4_0, 11008, "Q4_0 4096x11008")):
            if name in hosts:
                log(f"cpu baseline {name}")
                cpus[name] = cpu_gemv(t, hosts[name], cols, label, budget_s=2.0)
        if gemm_host is not None:
            for m in (16, 128, 512):
                log(f"cpu baseline gemm m={m}")
                cpus[f"q8_0_gemm_bf16_m{m}_4096x4096"] = cpu_gemm(gemm_host, m, seed=8)
        for name in [k for k in hosts if "_gemm_" in k]:
            m = int(name.split("_m")[1].split("_")[0])
            if m > 128:
                continue  # the m = 128 line's rate stands for it (m mat-vecs each)
            log(f"cpu baseline {name}")
            tid = {"q4_k": syn.Q4_K, "q4_0": syn.Q4_0, "q5_k": syn.Q5_K, "q6_k": syn.Q6_K}[name[:4]]
            cpus[name] = cpu_gemm(hosts[name], m, seed=8, type_id=tid)
        if moe_inputs is not None:
            log("cpu baseline moe")
            cpus["moe_q4_k_e128_top8_t16"] = cpu_moe(*moe_inputs)
        # One shared description instead of a sample text per entry.
        for c in cpus.values():
            c.pop("sample", None)
        extra["cpu_baselines_note"] = (
            "oracle (C restatement of the reference Java raw route) on all host cores with the "
            "reference's row chunking; GEMV: the full matrix, median of >= 10 reps after 2 "
            "warm-ups; GEMM: m mat-vecs (the reference's prefill); MoE: every route's expert "
            "mat-vecs per route, as the reference runs them")
        extra["cpu_baselines"] = cpus

    ms = head["ms_per_step"]
    value = head["weight_gbs"]
    achieved = head["algo_gbs"]
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": args.warmup,
        "device_warmup_s": round(warmed, 2),
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded; GGUF Q4_K packed weights, fp32 N(0,1) activation)",
        "config": {
            "workload": "q4_k_gemv_m1_k4096_n14336",
            "type": "Q4_K", "m": 1, "k": 4096, "n": 14336,
            "weight_bytes": head["weight_bytes"], "weight_copies": head["weight_copies"],
            "prepared_layout": head["prepared_layout"],
            "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(),
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    g512 = extra.get("q8_0_gemm_bf16_m512_4096x4096")
    if g512:
        line["gemm_tflops_m512"] = round(g512["tflops"], 2)
    # Last key: one short entry per configuration, so that the end of the
    # line (what a log tail keeps) carries every configuration's figure.
    line["configs"] = config_summary(head, extra, cpu)
    print(json.dumps(_rounded(line)))
    return 0


# (summary name, extra key, roofline) for the configurations the metric and
# its five configurations name, in that order.
SUMMARY = (
    ("C0_q8_0_gemv_4096x4096", "q8_0_gemv_4096x4096", "hbm"),
    ("C1_q4_0_gemv_4096x11008", "q4_0_gemv_4096x11008", "hbm"),
    ("C2a_q4_k_gemv_4096x14336", None, "hbm"),
    ("C2b_q4_k_gemv_4096x128256", "q4_k_gemv_4096x128256", "hbm"),
    ("C3_gemm_m16", "q8_0_gemm_bf16_m16_4096x4096", "hbm"),
    ("C3_gemm_m128", "q8_0_gemm_bf16_m128_4096x4096", "both"),
    ("C3_gemm_m512", "q8_0_gemm_bf16_m512_4096x4096", "mfma"),
    ("C4_moe_e128_top8_t16", "moe_q4_k_e128_top8_t16", "hbm"),
)


def config_summary(head, extra, head_cpu=None):
    """Per configuration: microseconds per launch, the fraction of the
    roofline that bounds it (HBM 8 TB/s on algorithmic bytes, or dense bf16
    MFMA 2.5 PFLOP/s) and the CPU baseline's rate where one was measured."""
    cpus = extra.get("cpu_baselines", {})
    out = {}
    for name, key, bound in SUMMARY:
        r = head if key is None else extra.get(key)
        if not r:
            continue
        e = {"us": round(r["ms_per_step"] * 1e3, 2)}
        if bound in ("hbm", "both"):
            e["hbm_frac"] = round(r["algo_gbs"] / HBM_PEAK_GBS, 3)
        if bound in ("mfma", "both"):
            e["mfma_frac"] = round(r["mfma_frac"], 3)
            e["tflops"] = round(r["tflops"], 1)
        c = cpus.get(key) if key is not None else head_cpu
        if c:
            e["cpu"] = f"{c['value']:.1f} {c['unit'].split(' ')[0]}"
        out[name] = e
    return out


def _rounded(obj):
    """Floats to 4 significant digits (the timing noise is larger), so that
    the one JSON line stays short."""
    if isinstance(obj, float):
        return float(f"{obj:.4g}") if math.isfinite(obj) else obj
    if isinstance(obj, dict):
        return {k: _rounded(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return [_rounded(v) for v in obj]
    return obj


def _has_symbol(name: str) -> bool:
    from gollek_amd import _native
    return hasattr(_native.load(), name)


if __name__ == "__main__":
    sys.exit(main())
