"""Benchmark of the vortx linalg hot path on one MI355X.

Headline (BASELINE.json metric, first named config): Q4_0 GEMV y = W x,
W 11008 x 4096, batch 1, throughput in GB/s of algorithmic bytes
(M * K/32 * 18 + 4 K + 4 M per launch). One step = one GEMV launch over the
next of >= 512 MB of distinct weight copies (so the 256 MB Infinity Cache
cannot serve them), inputs resident in HBM before timing starts.

Secondary lines in the same JSON object: the other BASELINE GEMV configs
(Q8_0 4096 x 4096 b=1 and b=8, Q4_K 32000 x 4096 and 14336 x 4096 b=1,
Q4_0 4096 x 11008 b=1, b=4 and b=8, Q4_0 11008 x 4096 b=4 and b=8, Q4_K
14336 x 4096 and 32000 x 4096 b=16; GB/s of algorithmic bytes), the f32
GEMV 11008 x 4096 and the same kernel as a read-only stream at the
headline's size and at 537 MB, the contiguous copy of a transposed
8192^2 view and a plain streaming copy of a contiguous one (the achievable
bandwidth beside the 8 TB/s peak), the same streaming copy at the headline's
size (25.4 MB per launch, graph-replayed: the achievable rate of one launch
that small), the Q8_0 and Q4_K quantizers on 14336 x 4096, the GGUF file
-> HBM upload (against the PCIe 5.0 x16 link) and the f32 GEMMs 4096^3,
4096 x 11008 x 4096, 4096^3 with a transposed-B view and the broadcast
batch (TFLOP/s), and the reference's GEMM size sweep (64..4096, tiled and
naive), each with its roofline, plus CPU baselines from the
oracle's OpenMP restatements on the host cores.

Timing: `value` is whole-job throughput: K steps replayed from a HIP graph
(captured eager launches) between two synchronizations (wall clock).
`roofline.achieved` divides the algorithmic bytes (or flops) of one launch
by the kernel's average launch duration: HIP events recorded on the stream
the kernels run on, bracketing the same timed region, divided by the number
of launches. rocprofv3 summaries of the same command are kept under
profiles/.

Usage: python bench.py [--gpus 1] [--steps 2000] [--warmup 200]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, public spec
F32_MFMA_PEAK_TFS = 157.3   # MI355X dense f32 matrix, public spec
PCIE_PEAK_GBS = 64.0        # host link: PCIe 5.0 x16, one direction
METRIC = "Q4_0/Q8_0 GEMV HBM GB/s at 11008x4096 b=1; f32 GEMM TFLOP/s at 4096^3"
# What the default GEMV path computes in: x split per 32-element block into two
# int8 levels with one f32 scale, products and block sums with the exactly
# decoded weights in int32, scaling and accumulation in f32.
DT_INT8X = "int8 x int4/int8 -> int32, f32 scale and accumulate"
X_REPR = ("x rounded per 32-element block to c (254 x1 + x2), x1 and x2 int8, c ~ max|x_blk| / 32000: "
          "|error| <= c / 2 ~ 1.6e-5 max|x_blk| per element")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def gemv_bytes(qtype: int, M: int, K: int, B: int) -> int:
    from vortx_amd.synthetic import row_bytes
    return M * row_bytes(qtype, K) + 4 * B * K + 4 * B * M


def load_traffic(name: str):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/*.json)."""
    p = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    return None


def graph_time(launch, steps: int):
    """Capture min(steps, 500) launches (launch(i, stream)) into a HIP graph
    on a side stream and replay it steps // that many times between two
    synchronizations. Returns (launches done, wall seconds, HIP-event ms on
    the stream the kernels run on)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    chunk = min(steps, 500)
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            for i in range(chunk):
                launch(i, s)
    torch.cuda.synchronize()
    reps = max(1, steps // chunk)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):  # replay() launches on the current stream
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(s)
        for _ in range(reps):
            graph.replay()
        e1.record(s)
        torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return reps * chunk, wall, e0.elapsed_time(e1)


def time_gemv(qtype: int, M: int, K: int, B: int, steps: int, warmup: int, label: str, x_f32: bool = False):
    """One step = vx_gemv_q on the next of >= 512 MB of weight copies
    (K launches captured into a HIP graph and replayed; HIP events on the
    graph's stream bracket the timed region). At B >= 2 on the default int8-x
    path a step is two launches (vx_quantize_x, then vx_gemv_xq); the GEMV
    kernel is then also timed alone, on a ready split, for the roofline."""
    import torch

    import vortx_amd as vx
    from vortx_amd import synthetic as S

    dev = torch.device("cuda:0")
    nbytes = M * S.row_bytes(qtype, K)
    ncopy = max(2, -(-(512 << 20) // nbytes) + 1)
    log(f"[{label}] generating {ncopy} weight copies ({ncopy * nbytes / 2**20:.0f} MiB)")
    log(f"[copies] {ncopy} x {nbytes}")
    distinct = [S.quant_weights(qtype, M, K, seed=100 + i, device=dev) for i in range(min(4, ncopy))]
    ws = [distinct[i % len(distinct)].clone() for i in range(ncopy)]
    del distinct
    x = S.activations(B, K, seed=7, device=dev)
    y = torch.empty((B, M), device=dev)
    g = vx.QuantGemv(0)
    qws = [vx.QWeight(w, qtype, M, K) for w in ws]
    xv, yv = x.t(), y.t()

    for i in range(warmup):
        g.dispatch(yv, qws[i % ncopy], xv, x_f32=x_f32)
    torch.cuda.synchronize()
    done, wall, ev_ms = graph_time(lambda i, s: g.dispatch(yv, qws[i % ncopy], xv, stream=s, x_f32=x_f32), steps)
    alg = gemv_bytes(qtype, M, K, B)
    r = {"steps": done, "ms_per_step": wall * 1e3 / done, "value": alg * done / wall / 1e9,
         "avg_launch_ms": ev_ms / done, "alg_bytes": alg, "weight_copies": ncopy, "launches_per_step": 1}
    # the library splits x inside the GEMV kernels (one launch) for 2 <= B <= 8
    # with K <= 4096 and x of stride 1 along K (as here); otherwise a step is
    # vx_quantize_x + vx_gemv_xq
    fused = 2 <= B <= 8 and K <= 4096
    if B >= 2 and not x_f32 and not fused:
        q = vx.XQ.empty(K, B)
        g.quantize_x(q, xv)
        for i in range(min(warmup, 20)):
            g.dispatch_xq(yv, qws[i % ncopy], q)
        torch.cuda.synchronize()
        n2, _, ev2 = graph_time(lambda i, s: g.dispatch_xq(yv, qws[i % ncopy], q, stream=s), steps)
        r["launches_per_step"] = 2
        r["step_ms_events"] = r["avg_launch_ms"]
        r["avg_launch_ms"] = ev2 / n2  # the dominant kernel (vx_gemv_xq) alone
    return r


def time_gemv_f32(M: int, K: int, steps: int, warmup: int):
    """f32 GEMV y = A x (the GEMM op's N == 1 route, vx_gemv_f32): A [M, K]
    row-major f32 read once, so 4 M K + 4 K + 4 M algorithmic bytes per launch;
    A rotating over >= 512 MB of copies, K launches captured into a HIP graph
    and replayed as in time_gemv. A read-only HBM stream with one FMA per
    element: the achievable read rate of a launch that size."""
    import torch

    import vortx_amd as vx

    dev = torch.device("cuda:0")
    nbytes = 4 * M * K
    ncopy = max(2, -(-(512 << 20) // nbytes) + 1)
    log(f"[copies] {ncopy} x {nbytes}")
    base = [torch.randn((M, K), device=dev) for _ in range(min(4, ncopy))]
    As = [base[i % len(base)].clone() if i >= len(base) else base[i] for i in range(ncopy)]
    x = torch.randn((K, 1), device=dev)
    y = torch.empty((M, 1), device=dev)
    gm = vx.Gemm(0)
    for i in range(warmup):
        gm.dispatch(y, As[i % ncopy], x)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    chunk = min(steps, 500)
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            for i in range(chunk):
                gm.dispatch(y, As[i % ncopy], x, stream=s)
    torch.cuda.synchronize()
    reps = max(1, steps // chunk)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(s)
        for _ in range(reps):
            graph.replay()
        e1.record(s)
        torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    done = reps * chunk
    alg = 4 * M * K + 4 * K + 4 * M
    return {"steps": done, "ms_per_step": wall * 1e3 / done, "value": alg * done / wall / 1e9,
            "avg_launch_ms": e0.elapsed_time(e1) / done, "alg_bytes": alg, "copies": ncopy}


def time_gemm_sweep(dims=(64, 128, 256, 512, 768, 1024, 1536, 2048, 4096)):
    """The reference's GEMM benchmark (examples/gemm_bench.rs): square f32
    GEMMs of each size, 3 warmup + 10 timed launches of the default (tiled)
    route and of the naive kernel, average launch time from HIP events."""
    import torch

    import vortx_amd as vx
    from vortx_amd import synthetic as S

    dev = torch.device("cuda:0")
    gm = vx.Gemm(0)
    pts = []
    for d in dims:
        a = S.uniform((d, d), 1, dev)
        b = S.uniform((d, d), 2, dev)
        c = torch.empty((d, d), device=dev)
        row = {"dim": d}
        for name, fn in (("tiled", gm.dispatch), ("naive", gm.dispatch_naive)):
            for _ in range(3):
                fn(c, a, b)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(10):
                fn(c, a, b)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / 10
            row[f"{name}_ms"] = ms
            row[f"{name}_tflops"] = 2.0 * d ** 3 / (ms * 1e-3) / 1e12
        row["speedup"] = row["naive_ms"] / row["tiled_ms"]
        pts.append(row)
        log(f"[gemm_sweep] {row}")
    return pts


def time_gemm(M: int, N: int, K: int, steps: int, warmup: int, transb: bool = False):
    """C = A B with row-major A [M, K]; B is row-major [K, N], or with transb the
    stride-swapped view of an [N, K] buffer (the reference's transposed-B case)."""
    import torch

    import vortx_amd as vx
    from vortx_amd import synthetic as S

    dev = torch.device("cuda:0")
    a = S.uniform((M, K), 1, dev)
    b = S.uniform((N, K), 2, dev).t() if transb else S.uniform((K, N), 2, dev)
    c = torch.empty((M, N), device=dev)
    gm = vx.Gemm(0)
    for _ in range(warmup):
        gm.dispatch(c, a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        gm.dispatch(c, a, b)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launch_ms = e0.elapsed_time(e1) / steps
    flops = 2.0 * M * N * K
    return {"value": flops * steps / wall / 1e12, "avg_launch_ms": launch_ms, "flops": flops,
            "ms_per_step": wall * 1e3 / steps}


def time_gemm_broadcast(B: int, M: int, N: int, K: int, steps: int, warmup: int):
    """vx_gemm_f32_ex: out[b] = A[b] W + 1.0 * out[b] for a batch of B
    activations A [B, M, K] sharing one W [K, N] (broadcast batch dim) with
    the beta = 1 epilogue (C read and written): 2 B M N K flops."""
    import torch

    import vortx_amd as vx
    from vortx_amd import synthetic as S

    dev = torch.device("cuda:0")
    a = S.uniform((B, M, K), 3, dev)
    w = S.uniform((K, N), 4, dev)
    c = torch.zeros((B, M, N), device=dev)
    gm = vx.Gemm(0)
    for _ in range(warmup):
        gm.dispatch_ex(c, a, w, alpha=1.0, beta=1.0, broadcast=True)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        gm.dispatch_ex(c, a, w, alpha=1.0, beta=1.0, broadcast=True)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    flops = 2.0 * B * M * N * K
    return {"value": flops * steps / wall / 1e12, "avg_launch_ms": e0.elapsed_time(e1) / steps, "flops": flops,
            "ms_per_step": wall * 1e3 / steps}


def time_copy_like_gemv(nelem: int, steps: int, warmup: int):
    """The achievable bandwidth of ONE launch as large as the headline GEMV:
    Contiguous::launch of a contiguous f32 view of nelem elements (8 bytes
    per element, read + write), sources rotating over >= 512 MB, K launches
    captured into a HIP graph and replayed exactly as time_gemv does."""
    import torch

    import vortx_amd as vx

    dev = torch.device("cuda:0")
    shape = (nelem // 1024, 1024)
    nsrc = -(-(512 << 20) // (4 * nelem)) + 1
    srcs = [torch.randn(shape, device=dev) for _ in range(min(4, nsrc))]
    log(f"[copies] {nsrc} x {4 * shape[0] * shape[1]}")
    srcs = [srcs[i % len(srcs)].clone() for i in range(nsrc)]
    out = torch.empty(shape, device=dev)
    c = vx.Contiguous(0)
    for i in range(warmup):
        c.launch(out, srcs[i % nsrc])
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    chunk = min(steps, 500)
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            for i in range(chunk):
                c.launch(out, srcs[i % nsrc], stream=s)
    torch.cuda.synchronize()
    reps = max(1, steps // chunk)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(s)
        for _ in range(reps):
            graph.replay()
        e1.record(s)
        torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    done = reps * chunk
    nbytes = 8 * out.numel()
    return {"value": nbytes * done / wall / 1e9, "avg_launch_ms": e0.elapsed_time(e1) / done,
            "alg_bytes": nbytes, "ms_per_step": wall * 1e3 / done, "sources": nsrc}


def time_contiguous(shape, steps: int, warmup: int, transposed: bool = True):
    """vortx's Contiguous op (src/linalg/contiguous.rs) on a transposed f32
    view, or (transposed=False) on a contiguous one, where it is a plain
    streaming copy (the achievable-bandwidth reference): bytes = 8 per
    element (read + write); 4 rotating 256 MB sources."""
    import torch

    import vortx_amd as vx

    dev = torch.device("cuda:0")
    srcs = [torch.randn(shape, device=dev) for _ in range(4)]
    if transposed:
        srcs = [t.t() for t in srcs]
    out = torch.empty(srcs[0].shape, device=dev)
    c = vx.Contiguous(0)
    for i in range(warmup):
        c.launch(out, srcs[i % 4])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        c.launch(out, srcs[i % 4])
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    nbytes = 8 * out.numel()
    return {"value": nbytes * steps / wall / 1e9, "avg_launch_ms": e0.elapsed_time(e1) / steps,
            "alg_bytes": nbytes, "ms_per_step": wall * 1e3 / steps}


def time_quantize(qtype: int, M: int, K: int, steps: int, warmup: int):
    """ggml's reference quantizer (quantize_row_*_ref) of an f32 [M, K] matrix
    into blocks: bytes = 4 M K read + the blocks written; 2 rotating inputs of
    4 M K bytes each (>= 256 MB together at 14336x4096)."""
    import torch

    import vortx_amd as vx

    dev = torch.device("cuda:0")
    qk, bb = vx.qtype_info(qtype)
    xs = [torch.randn((M, K), device=dev) for _ in range(2)]
    buf = torch.empty(M * (K // qk) * bb, dtype=torch.uint8, device=dev)
    w = vx.QWeight(buf, qtype, M, K)
    qg = vx.QuantGemv(0)
    for i in range(warmup):
        qg.quantize(w, xs[i % 2])
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        qg.quantize(w, xs[i % 2])
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    nbytes = 4 * M * K + buf.numel()
    return {"value": nbytes * steps / wall / 1e9, "avg_launch_ms": e0.elapsed_time(e1) / steps,
            "alg_bytes": nbytes, "ms_per_step": wall * 1e3 / steps}


def time_gguf_upload(steps: int):
    """GGUF model file -> HBM (vx_gguf_upload) for a 1.14 GB file of four Q8_0
    65536x4096 tensors: parse, then the data section into a device buffer
    that was written once before (a fresh allocation's first write measures
    the device's page mapping, not the loader). The file sits in the page
    cache, as right after a download or a previous load."""
    import tempfile

    import numpy as np
    import torch

    import vortx_amd as vx
    from tests import gguf_writer as W

    K, M = 4096, 65536
    blob = np.random.default_rng(0).integers(0, 256, M * (K // 32) * 34, dtype=np.uint8).tobytes()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "bench.gguf")
        with open(path, "wb") as fh:
            fh.write(W.build([("general.architecture", W.STRING, "llama")],
                             [(f"blk.{i}.ffn_up.weight", [K, M], 8, blob) for i in range(4)]))
        del blob
        t0 = time.perf_counter()
        f = vx.GGUFFile(path)
        open_ms = (time.perf_counter() - t0) * 1e3
        n = f.header["data_size"]
        ctx = vx.QuantGemv(0)
        buf = torch.zeros(n, dtype=torch.uint8, device="cuda:0")
        f.upload(ctx, buf)
        times = []
        for _ in range(steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            f.upload(ctx, buf)
            times.append(time.perf_counter() - t0)
        f.close()
    times.sort()
    med = times[len(times) // 2]
    return {"value": n / med / 1e9, "bytes": n, "ms_per_step": med * 1e3, "open_ms": open_ms}


def cpu_baselines(threads: int):
    """Oracle OpenMP restatements on the host cores (bounded samples)."""
    import numpy as np

    from oracle import oracle as O
    from vortx_amd import synthetic as S

    out = {}
    bind = f"; OMP_PROC_BIND={os.environ.get('OMP_PROC_BIND', 'unset')}"
    M, K = 11008, 4096
    w = S.quant_weights(O.Q4_0, M, K, seed=100).numpy()
    x = S.activations(1, K, seed=7).numpy()
    O.gemv_q_f32_omp(O.Q4_0, w, M, K, x, threads)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 10.0:
        O.gemv_q_f32_omp(O.Q4_0, w, M, K, x, threads)
        n += 1
    dt = (time.perf_counter() - t0) / n
    out["q4_0"] = {"value": gemv_bytes(2, M, K, 1) / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
                   "sample": f"{n} x Q4_0 GEMV 11008x4096 b=1 on one 25 MB matrix (oracle gemv_q_f32_omp, "
                             f"builder's dequant-dot restatement; the reference has no quantized path){bind}"}
    a = np.random.default_rng(1).uniform(-1, 1, (1024, 1024)).astype(np.float32)
    b = np.random.default_rng(2).uniform(-1, 1, (1024, 1024)).astype(np.float32)
    for _ in range(3):  # examples/gemm_bench.rs:11-12: 3 warmup + 10 timed
        O.gemm_tiled_f32_omp(a, b, threads)
    t0 = time.perf_counter()
    for _ in range(10):
        O.gemm_tiled_f32_omp(a, b, threads)
    dt = (time.perf_counter() - t0) / 10
    out["gemm1024"] = {"value": 2.0 * 1024 ** 3 / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
                       "sample": "10 timed (3 warmup) f32 GEMM 1024^3, OpenMP restatement of gemm_tiled "
                                 f"(64x64x16 tiles, reference k order){bind}"}
    for M, N, K, key in ((4096, 4096, 4096, "gemm4096"), (4096, 11008, 4096, "gemm4096x11008")):
        a = np.random.default_rng(1).uniform(-1, 1, (M, K)).astype(np.float32)
        b = np.random.default_rng(2).uniform(-1, 1, (K, N)).astype(np.float32)
        O.gemm_tiled_f32_omp(a, b, threads)  # 1 warmup + 3 timed for the 4096-class shapes
        t0 = time.perf_counter()
        for _ in range(3):
            O.gemm_tiled_f32_omp(a, b, threads)
        dt = (time.perf_counter() - t0) / 3
        out[key] = {"value": 2.0 * M * N * K / dt / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
                    "sample": f"3 timed (1 warmup) f32 GEMM {M}x{N}x{K}, OpenMP restatement of gemm_tiled "
                              f"(64x64x16 tiles, reference k order){bind}"}
    return out


def cpu_baselines_child(threads: int):
    """cpu_baselines in a child process of its own (no GPU use there), with
    its OpenMP threads pinned close together (OMP_PROC_BIND=close): pinning
    in this process would bind the main thread, and with it the GGUF upload's
    reader threads, to one core."""
    import subprocess
    env = dict(os.environ, OMP_PROC_BIND=os.environ.get("OMP_PROC_BIND", "close"), OMP_NUM_THREADS=str(threads))
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-baseline-only", str(threads)], env=env,
                       stdout=subprocess.PIPE, check=True, text=True)
    return json.loads(r.stdout.strip().splitlines()[-1])


# Batched and secondary GEMV configs: key -> (qtype, M, K, B, workload).
GEMV_SECONDARY = {
    "gemv_q8_0_4096x4096_b1": (8, 4096, 4096, 1, "Q8_0 GEMV 4096x4096 batch 1"),
    "gemv_q4_k_32000x4096_b1": (12, 32000, 4096, 1, "Q4_K GEMV 32000x4096 batch 1"),
    "gemv_q4_0_4096x11008_b1": (2, 4096, 11008, 1, "Q4_0 GEMV 4096x11008 batch 1"),
    "gemv_q4_k_14336x4096_b1": (12, 14336, 4096, 1, "Q4_K GEMV 14336x4096 batch 1"),
    "gemv_q4_0_11008x4096_b4": (2, 11008, 4096, 4, "Q4_0 GEMV 11008x4096 batch 4"),
    "gemv_q4_0_11008x4096_b8": (2, 11008, 4096, 8, "Q4_0 GEMV 11008x4096 batch 8"),
    "gemv_q4_0_4096x11008_b4": (2, 4096, 11008, 4, "Q4_0 GEMV 4096x11008 batch 4"),
    "gemv_q4_0_4096x11008_b8": (2, 4096, 11008, 8, "Q4_0 GEMV 4096x11008 batch 8"),
    "gemv_q8_0_4096x4096_b8": (8, 4096, 4096, 8, "Q8_0 GEMV 4096x4096 batch 8"),
    "gemv_q4_k_14336x4096_b16": (12, 14336, 4096, 16, "Q4_K GEMV 14336x4096 batch 16"),
    "gemv_q4_k_32000x4096_b16": (12, 32000, 4096, 16, "Q4_K GEMV 32000x4096 batch 16"),
}
GEMMS = {  # key -> (M, N, K, transb, workload)
    "gemm_f32_4096": (4096, 4096, 4096, False, "f32 GEMM 4096^3 (row-major A, B)"),
    "gemm_f32_4096x11008x4096": (4096, 11008, 4096, False, "f32 GEMM M=4096 N=11008 K=4096 (row-major A, B)"),
    "gemm_f32_4096_transb": (4096, 4096, 4096, True, "f32 GEMM 4096^3, B a transposed view of a row-major [N, K] buffer"),
}
# every workload in run order (the keys --only selects from)
KEYS = (["gemv_q4_0_11008x4096_b1", "gemv_q4_0_11008x4096_b1_f32x"] + list(GEMV_SECONDARY) +
        ["gemv_f32_11008x4096", "gemv_f32_1552x4096", "gemv_f32_32768x4096", "gemm_sweep"] + list(GEMMS) +
        ["gemm_f32_broadcast_8x1024", "contiguous_t8192", "copy_8192", "copy_3104x1024", "quantize_q8_0_14336x4096",
         "quantize_q4_k_14336x4096", "gguf_upload"])


def run_workloads(keys, steps: int, warmup: int) -> dict:
    """Run the named workloads in KEYS order; returns key -> result."""
    out = {}
    gsteps, gwarm = max(5, min(50, steps // 40)), max(2, warmup // 100)
    for k in [k for k in KEYS if k in keys]:
        if k == "gemv_q4_0_11008x4096_b1":
            r = time_gemv(2, 11008, 4096, 1, steps, warmup, "q4_0")
        elif k == "gemv_q4_0_11008x4096_b1_f32x":
            # the headline config with x kept in f32 (VX_GEMV_X_F32): f32 FMA on
            # the exactly decoded weights, the exact-arithmetic twin of the default
            r = time_gemv(2, 11008, 4096, 1, steps, warmup, "q4_0_f32x", x_f32=True)
        elif k in GEMV_SECONDARY:
            qt, M, K, B, _ = GEMV_SECONDARY[k]
            r = time_gemv(qt, M, K, B, max(100, steps // (2 if B > 1 or M > 20000 else 1)), warmup, k)
        elif k == "gemv_f32_11008x4096":
            r = time_gemv_f32(11008, 4096, max(100, steps // 4), warmup)
        elif k == "gemv_f32_1552x4096":
            # a read-only stream of the headline's size: 1552 x 4096 f32 = 25.43 MB
            # (the Q4_0 GEMV moves 25.42 MB)
            r = time_gemv_f32(1552, 4096, steps, warmup)
        elif k == "gemv_f32_32768x4096":
            r = time_gemv_f32(32768, 4096, max(50, steps // 20), max(5, warmup // 20))
        elif k == "gemm_sweep":
            r = time_gemm_sweep()
        elif k in GEMMS:
            M, N, K, tb, _ = GEMMS[k]
            r = time_gemm(M, N, K, gsteps, gwarm, transb=tb)
        elif k == "gemm_f32_broadcast_8x1024":
            r = time_gemm_broadcast(8, 1024, 4096, 4096, gsteps, gwarm)
        elif k == "contiguous_t8192":
            r = time_contiguous((8192, 8192), max(10, steps // 20), 5)
        elif k == "copy_8192":
            r = time_contiguous((8192, 8192), max(10, steps // 20), 5, transposed=False)
        elif k == "copy_3104x1024":
            # one launch moving the headline GEMV's bytes (25,422,848 / 8 elements,
            # rounded up to whole rows of 1024)
            r = time_copy_like_gemv(3104 * 1024, steps, warmup)
        elif k == "quantize_q8_0_14336x4096":
            r = time_quantize(8, 14336, 4096, max(10, steps // 20), 3)
        elif k == "quantize_q4_k_14336x4096":
            r = time_quantize(12, 14336, 4096, max(10, steps // 100), 3)
        else:  # gguf_upload
            r = time_gguf_upload(5)
        log(f"[{k}] {r}")
        out[k] = r
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", metavar="KEYS",
                    help="comma-separated workload keys (profiling runs): print their raw results, not the "
                         "benchmark line; keys: " + ", ".join(KEYS))
    ap.add_argument("--cpu-baseline-only", type=int, default=0, metavar="THREADS",
                    help=argparse.SUPPRESS)  # the CPU leg's own process: print its JSON and exit
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the hot path shards by output rows; see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        return 2

    if args.cpu_baseline_only:
        print(json.dumps(cpu_baselines(args.cpu_baseline_only)), flush=True)
        return 0
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if args.only:
        keys = [k for k in args.only.split(",") if k]
        bad = [k for k in keys if k not in KEYS]
        if bad:
            print(f"unknown workload keys {bad}; known: {KEYS}", file=sys.stderr)
            return 2
        print(json.dumps({"only": run_workloads(keys, args.steps, args.warmup)}), flush=True)
        return 0

    R = run_workloads(KEYS, args.steps, args.warmup)
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    cpu = None if args.no_cpu else cpu_baselines_child(threads)
    if cpu:
        log(f"[cpu] {cpu}")

    def roof_hbm(key):
        r = R[key]
        achieved = r["alg_bytes"] / (r["avg_launch_ms"] * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": achieved / HBM_PEAK_GBS, "traffic": load_traffic(key)}

    def roof_mfma(key):
        r = R[key]
        achieved = r["flops"] / (r["avg_launch_ms"] * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": achieved, "peak": F32_MFMA_PEAK_TFS, "unit": "TFLOP/s",
                "frac": achieved / F32_MFMA_PEAK_TFS, "traffic": load_traffic(key)}

    def gemv_line(key, workload, dtype):
        r = R[key]
        d = {"workload": workload, "value": r["value"], "unit": "GB/s", "ms_per_step": r["ms_per_step"],
             "dtype": dtype, "roofline": roof_hbm(key)}
        if r.get("launches_per_step", 1) == 2:
            d["launches_per_step"] = 2
            d["note"] = ("a step is vx_quantize_x + vx_gemv_xq; roofline.achieved divides the step's algorithmic "
                         "bytes by vx_gemv_xq's own average duration (graph-replayed alone on a ready split), "
                         "roofline.traffic is both kernels' HBM bytes per step")
        elif key in GEMV_SECONDARY and GEMV_SECONDARY[key][3] >= 2:
            d["note"] = "one launch per step: the batched GEMV kernel splits x itself"
        return d

    q40 = R["gemv_q4_0_11008x4096_b1"]
    sweep = R["gemm_sweep"]
    gg = R["gguf_upload"]
    line = {
        "metric": METRIC,
        "value": q40["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": q40["steps"],
        "warmup": args.warmup,
        "ms_per_step": q40["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DT_INT8X,
        "data": "synthetic",
        "config": {"workload": "Q4_0 GEMV y=Wx, W 11008x4096 (GGML Q4_0 blocks), batch 1",
                   "M": 11008, "K": 4096, "batch": 1, "weight_copies": q40["weight_copies"],
                   "bytes_per_step": q40["alg_bytes"], "timing": "HIP-graph replay of eager launches",
                   "x_repr": X_REPR},
        "roofline": roof_hbm("gemv_q4_0_11008x4096_b1"),
        "cpu_baseline": cpu["q4_0"] if cpu else None,
        "secondary": [
            gemv_line("gemv_q4_0_11008x4096_b1_f32x", "Q4_0 GEMV 11008x4096 batch 1, x kept in f32 (VX_GEMV_X_F32: "
                      "f32 FMA on the exactly decoded weights)", "f32"),
        ] + [gemv_line(k, v[4], DT_INT8X) for k, v in GEMV_SECONDARY.items()] + [
            gemv_line("gemv_f32_11008x4096", "f32 GEMV y = A x, A 11008x4096 row-major (the GEMM op's N == 1 route, "
                      "vx_gemv_f32), A rotating over >= 512 MB, HIP-graph replay", "f32"),
            gemv_line("gemv_f32_1552x4096", "read-only HBM stream of the headline's size: vx_gemv_f32 on A 1552x4096 "
                      "f32 (25.43 MB read per launch; the Q4_0 GEMV reads 25.42 MB), A rotating over >= 512 MB, "
                      "HIP-graph replay (the achievable read rate of one launch this size)", "f32"),
            gemv_line("gemv_f32_32768x4096", "read-only HBM stream, 537 MB per launch: vx_gemv_f32 on A 32768x4096 "
                      "f32 (the achievable read rate of a long stream)", "f32"),
            {"workload": "contiguous copy of a transposed 8192x8192 f32 view (Contiguous::launch)",
             "value": R["contiguous_t8192"]["value"], "unit": "GB/s",
             "ms_per_step": R["contiguous_t8192"]["ms_per_step"], "roofline": roof_hbm("contiguous_t8192")},
            {"workload": "streaming copy: Contiguous::launch of a contiguous 8192x8192 f32 view (achievable HBM "
                         "bandwidth of a plain read + write stream on this GPU)",
             "value": R["copy_8192"]["value"], "unit": "GB/s", "ms_per_step": R["copy_8192"]["ms_per_step"],
             "roofline": roof_hbm("copy_8192")},
            {"workload": "streaming copy of the headline's size: Contiguous::launch of a contiguous 3104x1024 f32 "
                         "view, 25.43 MB read + written per launch (the headline GEMV moves 25.42 MB), sources "
                         "rotating over >= 512 MB, HIP-graph replay (the achievable rate of one launch this size)",
             "value": R["copy_3104x1024"]["value"], "unit": "GB/s", "ms_per_step": R["copy_3104x1024"]["ms_per_step"],
             "roofline": roof_hbm("copy_3104x1024")},
        ] + [
            {"workload": f"quantize f32 14336x4096 to {label} blocks (ggml reference quantizer)",
             "value": R[k]["value"], "unit": "GB/s", "ms_per_step": R[k]["ms_per_step"], "roofline": roof_hbm(k),
             **({"note": "VALU-bound: ggml's 21-candidate scale/min search per 32-value sub-block, one "
                         "sub-block per lane, 11-13k VALU instructions per wave (ISA count): 0.53-0.59 ms at one "
                         "wave-instruction per CU per cycle (256 CUs, 2.4 GHz); the HBM fraction is not its bound"}
                if label == "Q4_K" else {})}
            for k, label in (("quantize_q8_0_14336x4096", "Q8_0"), ("quantize_q4_k_14336x4096", "Q4_K"))
        ] + [
            {"workload": "GGUF file (page cache) -> HBM upload, 1.14 GB data section (vx_gguf_upload)",
             "value": gg["value"], "unit": "GB/s", "ms_per_step": gg["ms_per_step"], "open_ms": gg["open_ms"],
             "roofline": {"bound": "pcie", "achieved": gg["value"], "peak": PCIE_PEAK_GBS, "unit": "GB/s",
                          "frac": gg["value"] / PCIE_PEAK_GBS, "traffic": None}},
        ] + [
            {"workload": v[4], "value": R[k]["value"], "unit": "TFLOP/s", "ms_per_step": R[k]["ms_per_step"],
             "roofline": roof_mfma(k),
             **({"cpu_baseline": cpu["gemm4096"], "cpu_baseline_1024": cpu["gemm1024"]} if cpu and k == "gemm_f32_4096"
                else {"cpu_baseline": cpu["gemm4096x11008"]} if cpu and k == "gemm_f32_4096x11008x4096" else {})}
            for k, v in GEMMS.items()
        ] + [
            {"workload": "broadcast f32 GEMM out[b] = A[b] W + out[b], A [8, 1024, 4096], shared W [4096, 4096] "
                         "(vx_gemm_f32_ex, beta = 1)", "value": R["gemm_f32_broadcast_8x1024"]["value"],
             "unit": "TFLOP/s", "ms_per_step": R["gemm_f32_broadcast_8x1024"]["ms_per_step"],
             "roofline": roof_mfma("gemm_f32_broadcast_8x1024")},
            {"workload": "f32 GEMM sweep of the reference's benchmark (examples/gemm_bench.rs: dim^3 for dim in "
                         "64..4096, 3 warmup + 10 timed launches each), default tiled route and naive kernel",
             "unit": "TFLOP/s", "value": sweep[-1]["tiled_tflops"], "points": sweep},
        ],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
