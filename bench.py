"""Benchmark of the vortx linalg hot path on one MI355X.

Headline (BASELINE.json metric, first named config): Q4_0 GEMV y = W x,
W 11008 x 4096, batch 1, throughput in GB/s of algorithmic bytes
(M * K/32 * 18 + 4 K + 4 M per launch). One step = one GEMV launch over the
next of >= 512 MB of distinct weight copies (so the 256 MB Infinity Cache
cannot serve them), inputs resident in HBM before timing starts.

Beside it, top-level objects for the metric's other halves and the
ceiling: Q8_0 4096 x 4096 b=1, the headline with x kept in f32, the read
probe (the headline GEMV's loads of W alone: the most its access pattern
can stream in one launch) and the f32 GEMM 4096^3 (TFLOP/s, 50 timed
launches after 50 warmups). Compact lines ([value, ms per step, roofline
achieved, roofline frac, launches per step]) cover the other BASELINE GEMV
configs, the activation split kernel alone, the f32 GEMV as a read-only
stream (headline size, 537 MB), copies (transposed 8192^2 view, contiguous
8192^2, one launch of the headline's 25.4 MB), the quantizers, the other
GEMM shapes and the broadcast batch; then the GGUF upload, the reference's
GEMM size sweep (examples/gemm_bench.rs: 64..4096, tiled and naive) and
CPU baselines from the oracle's OpenMP restatements on the host cores.

Timing: exactly K steps between two synchronizations; the timed region is
bracketed by HIP events recorded on the stream the kernels run on (timing-only
events: hipEventDisableSystemFence, so recording one flushes no caches), and
`ms_per_step` / `value` / `roofline.achieved` are that region's duration per
step and the algorithmic bytes (or flops) over it (a two-launch batched step
counts both launches; its GEMV kernel alone is reported as `gemv_only`). Up
to 256 steps (the headline at the driver's --steps 20) the launches are
issued directly on the stream behind a short spin kernel queued ahead of the
start event (the "blocking kernel" of NVBench), so the host has queued every
launch before the GPU reaches the start event and the region holds GPU time
only; each run checks that this held (the start event still pending once all
launches are queued) and otherwise retries with a longer spin. Longer runs,
and every other line (at least 1000 launches), replay HIP graphs of up to
500 captured launches (a graph replay carries ~9.5 us of its own on the GPU,
measured: at 20 launches per replay 0.47 us per step, at 500 0.02).
`wall_ms_per_step` is the wall clock between the two synchronizations per
step (host-side launches and synchronization included, the spin excluded).
rocprofv3 summaries of the same command are kept under profiles/. Nothing
goes to stderr without --verbose.

Usage: python bench.py [--gpus 1] [--steps 2000] [--warmup 200] [--verbose] [--only KEYS]
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


VERBOSE = False


def log(msg: str) -> None:
    """Progress on stderr, only with --verbose (the driver keeps the tail of
    the output, which must hold the whole JSON line)."""
    if VERBOSE:
        print(msg, file=sys.stderr, flush=True)


def rnd(v, sig: int = 4):
    """v rounded to `sig` significant digits (compact JSON)."""
    if v is None or isinstance(v, (bool, int, str)):
        return v
    return float(f"{v:.{sig}g}")


def gemv_bytes(qtype: int, M: int, K: int, B: int) -> int:
    from vortx_amd.synthetic import row_bytes
    return M * row_bytes(qtype, K) + 4 * B * K + 4 * B * M


def load_traffic(name: str):
    """HBM bytes per launch (per step for two-launch lines) measured with
    rocprofv3 --pmc, kept in profiles/traffic_<name>.json."""
    p = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    return None


def per_step(done: int, wall: float, ev_ms: float, work: float, scale: float = 1e9) -> dict:
    """ms_per_step and value (work per step / scale per second) from the
    event-timed region, and the wall clock per step beside them."""
    ms = ev_ms / done
    return {"steps": done, "ms_per_step": ms, "step_ms_events": ms, "value": work / (ms * 1e-3) / scale,
            "wall_ms_per_step": wall * 1e3 / done}


EAGER_MAX = 256  # at most this many timed steps: direct launches behind a spin kernel


class HipEvent:
    """A timing-only HIP event (hipEventCreateWithFlags with
    hipEventDisableSystemFence) of the HIP runtime torch uses, recorded on a
    given stream. Recording it issues no system-scope cache writeback or
    invalidation, which a default event does and whose cost would fall inside
    a short timed region (same box, the headline at 20 steps: 6.32 us per
    step with torch's default events, 6.19 with these, mean of 6 pairs). The
    elapsed time is read only after a device synchronization."""
    DISABLE_SYSTEM_FENCE = 0x20000000
    NOT_READY = 600  # hipErrorNotReady
    _hip = None

    def __init__(self):
        import ctypes

        import torch  # noqa: F401  (its libamdhip64 is the one already loaded)

        if HipEvent._hip is None:
            HipEvent._hip = ctypes.CDLL("libamdhip64.so.7")
        self._c = ctypes
        self.h = ctypes.c_void_p()
        self._check(HipEvent._hip.hipEventCreateWithFlags(ctypes.byref(self.h),
                                                          ctypes.c_uint(self.DISABLE_SYSTEM_FENCE)))

    @staticmethod
    def _check(rc: int) -> None:
        if rc != 0:
            raise RuntimeError(f"HIP event call failed: hipError_t {rc}")

    def record(self, stream) -> None:
        self._check(HipEvent._hip.hipEventRecord(self.h, self._c.c_void_p(stream.cuda_stream)))

    def query(self) -> bool:
        rc = HipEvent._hip.hipEventQuery(self.h)
        if rc not in (0, self.NOT_READY):
            self._check(rc)
        return rc == 0

    def elapsed_time(self, end: "HipEvent") -> float:
        ms = self._c.c_float()
        self._check(HipEvent._hip.hipEventElapsedTime(self._c.byref(ms), self.h, end.h))
        return ms.value

    def __del__(self):
        # not during interpreter shutdown, when the HIP runtime may be gone
        if HipEvent._hip is not None and self.h and not sys.is_finalizing():
            HipEvent._hip.hipEventDestroy(self.h)


def graph_time(launch, steps: int):
    """Exactly `steps` launches (launch(i, stream)) on a side stream, timed by
    HIP events on that stream between two synchronizations (one untimed pass
    first). Up to EAGER_MAX steps: a spin kernel (torch.cuda._sleep), the
    start event, the launches, the end event, so that the host has queued
    every launch before the GPU reaches the start event; the start event still
    pending after the last launch is queued shows it (else the spin is made
    four times longer and the run repeated). Longer runs: HIP graphs of
    min(steps, 500) captured launches (the remainder in a second graph),
    replayed. Returns (launches done, wall seconds between the
    synchronizations less the spin, HIP-event ms of the timed launches)."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    e0, e1 = HipEvent(), HipEvent()
    if steps <= EAGER_MAX and hasattr(torch.cuda, "_sleep"):  # (a private torch helper: else graphs)
        es = HipEvent()
        with torch.cuda.stream(s):
            for i in range(steps):  # untimed pass
                launch(i, s)
        torch.cuda.synchronize()
        cycles = 4_000_000
        for _ in range(4):
            with torch.cuda.stream(s):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                es.record(s)
                torch.cuda._sleep(cycles)
                e0.record(s)
                for i in range(steps):
                    launch(i, s)
                covered = not e0.query()
                e1.record(s)
                torch.cuda.synchronize()
            wall = time.perf_counter() - t0 - es.elapsed_time(e0) * 1e-3
            if covered:
                break
            cycles *= 4
        else:
            raise RuntimeError("the spin kernel never outlasted the host's launches")
        return steps, max(wall, 0.0), e0.elapsed_time(e1)
    chunk = min(steps, 500)
    reps, rem = divmod(steps, chunk)
    graphs = []
    for n in (chunk, rem):
        if n:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                with torch.cuda.graph(g, stream=s):
                    for i in range(n):
                        launch(i, s)
            graphs.append(g)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):  # replay() launches on the current stream
        graphs[0].replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(s)
        for _ in range(reps):
            graphs[0].replay()
        if rem:
            graphs[1].replay()
        e1.record(s)
        torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return steps, wall, e0.elapsed_time(e1)


def weight_copies(qtype: int, M: int, K: int, dev):
    """>= 512 MB of weight copies (twice the 256 MB Infinity Cache), four
    distinct seeds."""
    from vortx_amd import synthetic as S
    nbytes = M * S.row_bytes(qtype, K)
    ncopy = max(2, -(-(512 << 20) // nbytes) + 1)
    distinct = [S.quant_weights(qtype, M, K, seed=100 + i, device=dev) for i in range(min(4, ncopy))]
    return [distinct[i % len(distinct)].clone() for i in range(ncopy)]


def time_gemv(qtype: int, M: int, K: int, B: int, steps: int, warmup: int, label: str, x_f32: bool = False,
              probe: bool = False):
    """One step = vx_gemv_q_ws on the next of >= 512 MB of weight copies
    (launches captured into a HIP graph and replayed; HIP events on the
    graph's stream bracket the timed region). At B >= 2 on the int8 path, a
    shape the GEMV kernel cannot split x for is two launches per step
    (vx_quantize_x into the caller's workspace, then vx_gemv_xq); the GEMV
    kernel is then also timed alone on a ready split. probe: the read probe
    (vx_gemv_q_read_probe) over the same copies instead of the GEMV."""
    import torch

    import vortx_amd as vx
    from vortx_amd import synthetic as S

    dev = torch.device("cuda:0")
    ws = weight_copies(qtype, M, K, dev)
    ncopy = len(ws)
    log(f"[{label}] {ncopy} weight copies of {ws[0].numel()} B")
    x = S.activations(B, K, seed=7, device=dev)
    y = torch.empty((B, M), device=dev)
    g = vx.QuantGemv(0)
    qws = [vx.QWeight(w, qtype, M, K) for w in ws]
    xv, yv = x.t(), y.t()
    wsp = vx.QuantGemv.workspace(qws[0], B)
    if probe:
        yp = torch.empty(M, device=dev)
        fn = lambda i, s=None: g.read_probe(yp, qws[i % ncopy], stream=s)  # noqa: E731
    else:
        fn = lambda i, s=None: g.dispatch(yv, qws[i % ncopy], xv, stream=s, x_f32=x_f32, workspace=wsp)  # noqa: E731
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    done, wall, ev_ms = graph_time(fn, steps)
    alg = M * S.row_bytes(qtype, K) + 4 * M if probe else gemv_bytes(qtype, M, K, B)
    r = dict(per_step(done, wall, ev_ms, alg), alg_bytes=alg, weight_copies=ncopy, launches_per_step=1)
    # the library's route with a workspace (xq_fused_ok in vx_host.cpp): the
    # GEMV splits x itself (one launch) with one pass and one 256-weight item
    # per wave (B <= 16), two with B <= 8 or three with B <= 4, except two
    # column groups below M = 24576; otherwise the split goes to the
    # workspace first (two launches)
    ipr = (K // 64 + 3) // 4
    xmax = 1 if B > 8 else (3 if qtype == 2 else 2)
    xi = (ipr + 15) // 16
    fused = 2 <= B <= 16 and xi <= xmax and (xi == 1 or (B <= 8 and xi == 2) or B <= 4) and not (B > 8 and M < 24576)
    if B >= 2 and not x_f32 and not probe and not fused:
        q = vx.XQ.empty(K, B)
        g.quantize_x(q, xv)
        for i in range(min(warmup, 20)):
            g.dispatch_xq(yv, qws[i % ncopy], q)
        torch.cuda.synchronize()
        n2, _, ev2 = graph_time(lambda i, s: g.dispatch_xq(yv, qws[i % ncopy], q, stream=s), steps)
        r["launches_per_step"] = 2
        r["gemv_ms_events"] = ev2 / n2  # vx_gemv_xq alone, on a ready split
    return r


def time_launch_floor(steps: int, warmup: int):
    """An empty kernel on the batch-1 GEMV's grid (vx_launch_floor), captured
    into a HIP graph and replayed as in time_gemv: the fixed cost of one
    launch, which every step pays before any byte moves."""
    import torch

    import vortx_amd as vx

    g = vx.QuantGemv(0)
    for _ in range(warmup):
        g.launch_floor()
    torch.cuda.synchronize()
    done, wall, ev = graph_time(lambda i, s: g.launch_floor(stream=s), steps)
    return dict(per_step(done, wall, ev, 0.0))


def time_gemv_f32(M: int, K: int, steps: int, warmup: int):
    """f32 GEMV y = A x (the GEMM op's N == 1 route, vx_gemv_f32): A [M, K]
    row-major f32 read once, so 4 M K + 4 K + 4 M algorithmic bytes per launch;
    A rotating over >= 512 MB of copies, launches captured into a HIP graph
    and replayed as in time_gemv. A read-only HBM stream with one FMA per
    element: the achievable read rate of a launch that size."""
    import torch

    import vortx_amd as vx

    dev = torch.device("cuda:0")
    nbytes = 4 * M * K
    ncopy = max(2, -(-(512 << 20) // nbytes) + 1)
    base = [torch.randn((M, K), device=dev) for _ in range(min(4, ncopy))]
    As = [base[i % len(base)].clone() if i >= len(base) else base[i] for i in range(ncopy)]
    x = torch.randn((K, 1), device=dev)
    y = torch.empty((M, 1), device=dev)
    gm = vx.Gemm(0)
    for i in range(warmup):
        gm.dispatch(y, As[i % ncopy], x)
    torch.cuda.synchronize()
    done, wall, ev = graph_time(lambda i, s: gm.dispatch(y, As[i % ncopy], x, stream=s), steps)
    alg = 4 * M * K + 4 * K + 4 * M
    return dict(per_step(done, wall, ev, alg), alg_bytes=alg, copies=ncopy)


def event_time(fn, steps: int, warmup: int):
    """warmup eager calls, then `steps` timed ones between two
    synchronizations: (wall seconds, HIP-event ms on the current stream)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = HipEvent(), HipEvent()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return time.perf_counter() - t0, e0.elapsed_time(e1)


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
        row = [d]
        for fn in (gm.dispatch, gm.dispatch_naive):
            _, ev = event_time(lambda: fn(c, a, b), 10, 3)
            row.append(2.0 * d ** 3 / (ev / 10 * 1e-3) / 1e12)
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
    wall, ev = event_time(lambda: gm.dispatch(c, a, b), steps, warmup)
    flops = 2.0 * M * N * K
    return dict(per_step(steps, wall, ev, flops, 1e12), flops=flops)


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
    wall, ev = event_time(lambda: gm.dispatch_ex(c, a, w, alpha=1.0, beta=1.0, broadcast=True), steps, warmup)
    flops = 2.0 * B * M * N * K
    return dict(per_step(steps, wall, ev, flops, 1e12), flops=flops)


def time_copy_like_gemv(nelem: int, steps: int, warmup: int):
    """The achievable bandwidth of ONE launch as large as the headline GEMV:
    Contiguous::launch of a contiguous f32 view of nelem elements (8 bytes
    per element, read + write), sources rotating over >= 512 MB, launches
    captured into a HIP graph and replayed exactly as time_gemv does."""
    import torch

    import vortx_amd as vx

    dev = torch.device("cuda:0")
    shape = (nelem // 1024, 1024)
    nsrc = -(-(512 << 20) // (4 * nelem)) + 1
    srcs = [torch.randn(shape, device=dev) for _ in range(min(4, nsrc))]
    srcs = [srcs[i % len(srcs)].clone() for i in range(nsrc)]
    out = torch.empty(shape, device=dev)
    c = vx.Contiguous(0)
    for i in range(warmup):
        c.launch(out, srcs[i % nsrc])
    torch.cuda.synchronize()
    done, wall, ev = graph_time(lambda i, s: c.launch(out, srcs[i % nsrc], stream=s), steps)
    nbytes = 8 * out.numel()
    return dict(per_step(done, wall, ev, nbytes), alg_bytes=nbytes, sources=nsrc)


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
    it = iter(range(1 << 30))
    wall, ev = event_time(lambda: c.launch(out, srcs[next(it) % 4]), steps, warmup)
    nbytes = 8 * out.numel()
    return dict(per_step(steps, wall, ev, nbytes), alg_bytes=nbytes)


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
    it = iter(range(1 << 30))
    wall, ev = event_time(lambda: qg.quantize(w, xs[next(it) % 2]), steps, warmup)
    nbytes = 4 * M * K + buf.numel()
    return dict(per_step(steps, wall, ev, nbytes), alg_bytes=nbytes)


def time_quantize_x(K: int, B: int, steps: int, warmup: int):
    """vx_quantize_x alone (the split step of the two-launch batched GEMV):
    x [K, B] f32 read (4 B K), levels and scales written (vx_xq_size);
    launches captured into a HIP graph and replayed."""
    import torch

    import vortx_amd as vx
    from vortx_amd import synthetic as S

    dev = torch.device("cuda:0")
    x = S.activations(B, K, seed=7, device=dev)
    q = vx.XQ.empty(K, B)
    g = vx.QuantGemv(0)
    for _ in range(warmup):
        g.quantize_x(q, x.t())
    torch.cuda.synchronize()
    done, wall, ev = graph_time(lambda i, s: g.quantize_x(q, x.t(), stream=s), steps)
    nbytes = 4 * B * K + vx.xq_size(K, B)
    return dict(per_step(done, wall, ev, nbytes), alg_bytes=nbytes)


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


# GEMV configs beside the headline: key -> (qtype, M, K, B, workload).
GEMV_SECONDARY = {
    "gemv_q4_k_32000x4096_b1": (12, 32000, 4096, 1, "Q4_K 32000x4096 b=1"),
    "gemv_q4_0_4096x11008_b1": (2, 4096, 11008, 1, "Q4_0 4096x11008 b=1"),
    "gemv_q4_k_14336x4096_b1": (12, 14336, 4096, 1, "Q4_K 14336x4096 b=1"),
    "gemv_q4_0_11008x4096_b4": (2, 11008, 4096, 4, "Q4_0 11008x4096 b=4"),
    "gemv_q4_0_11008x4096_b8": (2, 11008, 4096, 8, "Q4_0 11008x4096 b=8"),
    "gemv_q4_0_4096x11008_b4": (2, 4096, 11008, 4, "Q4_0 4096x11008 b=4"),
    "gemv_q4_0_4096x11008_b8": (2, 4096, 11008, 8, "Q4_0 4096x11008 b=8"),
    "gemv_q8_0_4096x4096_b8": (8, 4096, 4096, 8, "Q8_0 4096x4096 b=8"),
    "gemv_q4_k_14336x4096_b16": (12, 14336, 4096, 16, "Q4_K 14336x4096 b=16"),
    "gemv_q4_k_32000x4096_b16": (12, 32000, 4096, 16, "Q4_K 32000x4096 b=16"),
}
GEMMS = {  # key -> (M, N, K, transb, workload)
    "gemm_f32_4096": (4096, 4096, 4096, False, "f32 GEMM 4096^3, row-major A and B"),
    "gemm_f32_4096x11008x4096": (4096, 11008, 4096, False, "f32 GEMM M=4096 N=11008 K=4096, row-major"),
    "gemm_f32_4096_transb": (4096, 4096, 4096, True, "f32 GEMM 4096^3, B a transposed view of an [N,K] buffer"),
}
# every workload in run order (the keys --only selects from)
KEYS = (["gemv_q4_0_11008x4096_b1", "gemv_q8_0_4096x4096_b1", "gemv_q4_0_11008x4096_b1_f32x",
         "read_q4_0_11008x4096", "read_q8_0_4096x4096", "launch_floor"] + list(GEMV_SECONDARY) +
        ["split_x_11008_b8", "split_x_4096_b16", "gemv_f32_11008x4096", "gemv_f32_1552x4096",
         "gemv_f32_32768x4096"] + list(GEMMS) +
        ["gemm_f32_broadcast_8x1024", "gemm_sweep", "contiguous_t8192", "copy_8192", "copy_3104x1024",
         "quantize_q8_0_14336x4096", "quantize_q4_k_14336x4096", "gguf_upload"])
# GEMMs: this many timed launches after this many warmups, whatever --steps is;
# 50 warmups (~50 ms at 4096^3) because after the idle gap of the workload's
# set-up the clocks need tens of ms to come back (10 warmups read 4096^3 at
# 136 TFLOP/s where a warm GPU runs it at 140)
GEMM_STEPS, GEMM_WARMUP = 50, 50


def run_workloads(keys, steps: int, warmup: int) -> dict:
    """Run the named workloads in KEYS order; returns key -> result. The
    headline takes exactly `steps` timed steps after `warmup`; the other lines
    take at least 1000 launches (GEMV-sized, graph-replayed) or 50 (GEMMs)."""
    out = {}
    many = max(1000, steps)
    for k in [k for k in KEYS if k in keys]:
        if k == "gemv_q4_0_11008x4096_b1":
            r = time_gemv(2, 11008, 4096, 1, steps, warmup, k)
        elif k == "gemv_q8_0_4096x4096_b1":
            r = time_gemv(8, 4096, 4096, 1, many, max(warmup, 50), k)
        elif k == "gemv_q4_0_11008x4096_b1_f32x":
            # the headline config with x kept in f32 (VX_GEMV_X_F32): f32 FMA on
            # the exactly decoded weights, the exact-arithmetic twin of the default
            r = time_gemv(2, 11008, 4096, 1, many, max(warmup, 50), k, x_f32=True)
        elif k == "read_q4_0_11008x4096":
            r = time_gemv(2, 11008, 4096, 1, many, max(warmup, 50), k, probe=True)
        elif k == "read_q8_0_4096x4096":
            r = time_gemv(8, 4096, 4096, 1, many, max(warmup, 50), k, probe=True)
        elif k == "launch_floor":
            r = time_launch_floor(many, 50)
        elif k in GEMV_SECONDARY:
            qt, M, K, B, _ = GEMV_SECONDARY[k]
            r = time_gemv(qt, M, K, B, many, max(warmup, 50), k)
        elif k == "split_x_11008_b8":
            r = time_quantize_x(11008, 8, many, 50)
        elif k == "split_x_4096_b16":
            r = time_quantize_x(4096, 16, many, 50)
        elif k == "gemv_f32_11008x4096":
            r = time_gemv_f32(11008, 4096, many, 50)
        elif k == "gemv_f32_1552x4096":
            # a read-only stream of the headline's size: 1552 x 4096 f32 = 25.43 MB
            # (the Q4_0 GEMV moves 25.42 MB)
            r = time_gemv_f32(1552, 4096, many, 50)
        elif k == "gemv_f32_32768x4096":
            r = time_gemv_f32(32768, 4096, 100, 5)
        elif k == "gemm_sweep":
            r = time_gemm_sweep()
        elif k in GEMMS:
            M, N, K, tb, _ = GEMMS[k]
            r = time_gemm(M, N, K, GEMM_STEPS, GEMM_WARMUP, transb=tb)
        elif k == "gemm_f32_broadcast_8x1024":
            r = time_gemm_broadcast(8, 1024, 4096, 4096, GEMM_STEPS, GEMM_WARMUP)
        elif k == "contiguous_t8192":
            r = time_contiguous((8192, 8192), 100, 5)
        elif k == "copy_8192":
            r = time_contiguous((8192, 8192), 100, 5, transposed=False)
        elif k == "copy_3104x1024":
            # one launch moving the headline GEMV's bytes (25,422,848 / 8 elements,
            # rounded up to whole rows of 1024)
            r = time_copy_like_gemv(3104 * 1024, many, 50)
        elif k == "quantize_q8_0_14336x4096":
            r = time_quantize(8, 14336, 4096, 100, 3)
        elif k == "quantize_q4_k_14336x4096":
            r = time_quantize(12, 14336, 4096, 20, 3)
        else:  # gguf_upload
            r = time_gguf_upload(5)
        log(f"[{k}] {r}")
        out[k] = r
    return out


def roof(r: dict, key: str, bound: str = "hbm") -> dict:
    """roofline object of one line: algorithmic bytes (flops) of a step over
    the step's HIP-event time (both launches of a two-launch step)."""
    t = r["step_ms_events"] * 1e-3
    if bound == "hbm":
        a, peak, unit = r["alg_bytes"] / t / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        a, peak, unit = r["flops"] / t / 1e12, F32_MFMA_PEAK_TFS, "TFLOP/s"
    tr = load_traffic(key)
    return {"bound": bound, "achieved": rnd(a), "peak": peak, "unit": unit, "frac": rnd(a / peak, 3),
            "traffic": int(tr) if tr else None}


def main() -> int:
    global VERBOSE
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--verbose", action="store_true", help="progress lines on stderr")
    ap.add_argument("--only", default="", metavar="KEYS",
                    help="comma-separated workload keys (profiling runs): print their raw results, not the "
                         "benchmark line; keys: " + ", ".join(KEYS))
    ap.add_argument("--cpu-baseline-only", type=int, default=0, metavar="THREADS",
                    help=argparse.SUPPRESS)  # the CPU leg's own process: print its JSON and exit
    args = ap.parse_args()
    VERBOSE = args.verbose
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the hot path shards by output rows). Run with --gpus 1.", file=sys.stderr)
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

    def gline(key: str, workload: str, unit: str = "GB/s", bound: str = "hbm") -> dict:
        r = R[key]
        d = {"workload": workload, "value": rnd(r["value"]), "unit": unit, "ms_per_step": rnd(r["ms_per_step"]),
             "roofline": roof(r, key, bound)}
        if r.get("launches_per_step", 1) == 2:
            # a two-launch step: the GEMV kernel alone (on a ready split) beside it
            g = r["gemv_ms_events"]
            d["launches"] = 2
            d["gemv_only"] = {"us": rnd(g * 1e3), "GB/s": rnd(r["alg_bytes"] / (g * 1e-3) / 1e9)}
        return d

    def short(key: str, unit: str = "GB/s", bound: str = "hbm") -> list:
        """[value, ms per step, roofline achieved, roofline frac, launches]"""
        r = R[key]
        ro = roof(r, key, bound)
        return [rnd(r["value"]), rnd(r["ms_per_step"]), ro["achieved"], ro["frac"], r.get("launches_per_step", 1)]

    q40 = R["gemv_q4_0_11008x4096_b1"]
    probe = R["read_q4_0_11008x4096"]
    floor = R["launch_floor"]
    gg = R["gguf_upload"]
    line = {
        "metric": METRIC,
        "value": rnd(q40["value"]),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": q40["steps"],
        "warmup": args.warmup,
        "ms_per_step": rnd(q40["ms_per_step"]),
        "wall_ms_per_step": rnd(q40["wall_ms_per_step"]),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": DT_INT8X,
        "data": "synthetic",
        "config": {"workload": "Q4_0 GEMV y=Wx, W 11008x4096 (GGML Q4_0 blocks), batch 1",
                   "M": 11008, "K": 4096, "batch": 1, "weight_copies": q40["weight_copies"],
                   "bytes_per_step": q40["alg_bytes"],
                   "timing": ("timing-only HIP events (hipEventDisableSystemFence) around exactly the timed steps; <= %d steps: direct launches queued behind a "
                              "spin kernel, else HIP-graph replay" % EAGER_MAX),
                   "x_repr": X_REPR},
        "roofline": roof(q40, "gemv_q4_0_11008x4096_b1"),
        "cpu_baseline": cpu["q4_0"] if cpu else None,
        "q8_0_b1": gline("gemv_q8_0_4096x4096_b1", "Q8_0 GEMV 4096x4096 b=1 (the metric's other format)"),
        "q4_0_b1_f32x": gline("gemv_q4_0_11008x4096_b1_f32x", "headline config, x kept in f32 (VX_GEMV_X_F32)"),
        "read_ceiling": dict(gline("read_q4_0_11008x4096", "vx_gemv_q_read_probe: the headline GEMV's loads of W "
                                   "alone (no x, no arithmetic), 25.4 MB"),
                             gemv_over_probe=rnd(q40["step_ms_events"] / probe["step_ms_events"], 3)),
        "read_ceiling_q8_0": gline("read_q8_0_4096x4096", "vx_gemv_q_read_probe on Q8_0 4096x4096"),
        # the fixed cost of one launch (empty kernel, same grid, graph-replayed),
        # and the headline's bytes over its step time minus that cost
        "launch_floor": {"us": rnd(floor["step_ms_events"] * 1e3, 3),
                         "headline_GBps_above_floor": rnd(q40["alg_bytes"] / ((q40["step_ms_events"] -
                                                                               floor["step_ms_events"]) * 1e-3) / 1e9)},
        "gemm_4096": dict(gline("gemm_f32_4096", GEMMS["gemm_f32_4096"][4], "TFLOP/s", "mfma"),
                          steps=GEMM_STEPS, warmup=GEMM_WARMUP,
                          cpu_baseline=cpu["gemm4096"] if cpu else None),
        # compact lines: key -> [value, ms per step, roofline achieved, roofline frac, launches per step]
        "lines_fields": ["value", "ms_per_step", "roof_achieved", "roof_frac", "launches"],
        "lines_gbs": {k: short(k) for k in GEMV_SECONDARY},
        "lines_gbs_other": {k: short(k) for k in ("split_x_11008_b8", "split_x_4096_b16", "gemv_f32_11008x4096",
                                                   "gemv_f32_1552x4096", "gemv_f32_32768x4096", "contiguous_t8192",
                                                   "copy_8192", "copy_3104x1024", "quantize_q8_0_14336x4096",
                                                   "quantize_q4_k_14336x4096")},
        "lines_tflops": {k: short(k, "TFLOP/s", "mfma") for k in ("gemm_f32_4096x11008x4096", "gemm_f32_4096_transb",
                                                                   "gemm_f32_broadcast_8x1024")},
        "gguf_upload": {"value": rnd(gg["value"]), "unit": "GB/s", "ms": rnd(gg["ms_per_step"]),
                        "pcie_frac": rnd(gg["value"] / PCIE_PEAK_GBS, 3)},
        "gemm_sweep": {"fields": ["dim", "tiled_tflops", "naive_tflops"],
                       "points": [[d, rnd(t, 3), rnd(n, 3)] for d, t, n in R["gemm_sweep"]]},
        "cpu_baselines": {k: {"value": rnd(v["value"]), "unit": v["unit"], "cores": v["cores"]}
                          for k, v in (cpu or {}).items() if k != "q4_0"},
    }
    print(json.dumps(line, separators=(",", ":")), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
