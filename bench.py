"""Benchmark: fused-kernel fp32 TFLOP/s and HBM GB/s (% of roofline) on 1x MI355X.

Headline workload: the largest configuration, C4,
``out = (silu(X @ W1) * (X @ W2)) @ W3`` with X 4096x4096, W1/W2 4096x11008,
W3 11008x4096 fp32 (std 1/sqrt(fan_in), seed 3) through the fusion pipeline:
4 kernels (X@W1, X@W2, the sigmoid chain, and (h1*s*h2)@W3 with the chain in
the A loader), 1.108 TFLOP of matmul work per step.

A *step* is one pass of the hot path over one batch with inputs already
resident in HBM: the workload's fused kernels launched back to back on the
shim's stream.  Before every timed step the 256 MiB Infinity Cache is
flushed by reading a 512 MiB scratch buffer (outside the timed bracket), so
nothing starts cache-warm.  Timing: stream markers (HIP events without the
system-scope fence) recorded before the first launch, between launches and
after the last, so one step yields the step time and each kernel's time.
Each kernel is first run (flush, launch) for at least 50 ms of its own GPU
time, so the clocks have settled before the timed steps.  ``value`` =
1.108 TFLOP / mean step time; ``roofline`` is the dominant kernel's (the one
taking the largest share of the step).

Also measured (``per_kernel``): C2 (one fused elementwise kernel), C3
softmax (4 kernels), the 4096^3 matmul, C4 literal and the fused diamond
variant, C5 attention (32 heads; each of the 5 per-head kernels launched
once for all heads, ``api.run_batch``), each kernel against its roofline.

``cpu_baseline``: the same C4 expression on the host's cores in float32 --
the CPU oracle's op table (``oracle/ir_eval.py``; elementwise ops split over
row blocks on a thread pool) with NumPy/OpenBLAS sgemm, and beside it
torch on the CPU -- both pinned to the same thread count; ``per_config``
does the same for every other configuration.  ``end_to_end``: ``api.run``
wall times for C2 and C3 (host transfers included).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c2|c3|c4|gemm|c5|copy|fragments|ceilings|sweep]
       [--no-extra] [--no-cpu] [--no-flush] [--calibrate-copy]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix


def source_sha16(source: str) -> str:
    """First 16 hex digits of the SHA-256 of a kernel's source as launched:
    ties a profile's counters to the exact kernel a bench line times."""
    import hashlib

    return hashlib.sha256(source.encode()).hexdigest()[:16]


class GpuSensors:
    """The GPU's clocks, board power and temperatures, found through its PCI
    bus id: hwmon's inputs and the current level of ``pp_dpm_sclk`` /
    ``pp_dpm_mclk`` (the line marked ``*``), sampled every ~1 ms by a
    background thread while ``with`` is active.  Everything is optional: on
    a machine without readable files the summary is None.  A sample covers
    whatever the GPU did in that millisecond: around the per-kernel timing
    loops that includes each launch's cache flush and host synchronisation,
    so short kernels' clock readings are averages with idle gaps, lower than
    the clock the kernel itself ran at (its MFMA rate bounds that from
    below); the C4 steps run back to back and are read cleanly."""

    FILES = {"sclk_mhz": ("freq1_input", 1e-6), "mclk_mhz": ("freq2_input", 1e-6),
             "power_w": ("power1_average", 1e-6), "power_input_w": ("power1_input", 1e-6),
             "temp_edge_c": ("temp1_input", 1e-3), "temp_junction_c": ("temp2_input", 1e-3),
             "temp_mem_c": ("temp3_input", 1e-3)}
    DPM = {"sclk_mhz": "pp_dpm_sclk", "mclk_mhz": "pp_dpm_mclk"}
    PERIOD_S = 0.001
    PCI_BUS_ID = ""  # the bench's GPU, set once the device is known

    def __init__(self, pci_bus_id: str = ""):
        import glob

        dev = f"/sys/bus/pci/devices/{(pci_bus_id or self.PCI_BUS_ID).lower()}"
        self.paths = {}
        for d in glob.glob(f"{dev}/hwmon/hwmon*"):
            for key, (fname, scale) in self.FILES.items():
                f = os.path.join(d, fname)
                if os.access(f, os.R_OK):
                    self.paths[key] = (f, scale)
        for key, fname in self.DPM.items():
            f = os.path.join(dev, fname)
            if key not in self.paths and os.access(f, os.R_OK):
                self.paths[key] = (f, None)
        self.samples = {k: [] for k in self.paths}
        self._stop = None

    @staticmethod
    def _dpm_mhz(text: str) -> float:
        """The current level of a pp_dpm_* table (``1: 2100Mhz *``)."""
        for line in text.splitlines():
            if line.strip().endswith("*"):
                return float(line.split(":", 1)[1].strip().rstrip("*").strip().lower().rstrip("mhz"))
        raise ValueError("no current level")

    def _read(self):
        for key, (f, scale) in self.paths.items():
            try:
                with open(f) as fh:
                    text = fh.read()
                self.samples[key].append(self._dpm_mhz(text) if scale is None else float(text.strip()) * scale)
            except (OSError, ValueError, IndexError):
                pass

    def __enter__(self):
        import threading

        if not self.paths:
            return self
        self._stop = threading.Event()

        def loop():
            while not self._stop.is_set():
                self._read()
                self._stop.wait(self.PERIOD_S)

        self._thread = threading.Thread(target=loop, daemon=True)
        self._thread.start()
        return self

    def __exit__(self, *exc):
        if self._stop is not None:
            self._stop.set()
            self._thread.join()
            self._read()  # the state as the timed work ends

    def summary(self) -> dict | None:
        out = {}
        for key, v in self.samples.items():
            if v:
                out[key] = {"min": round(min(v), 1), "mean": round(float(np.mean(v)), 1), "max": round(max(v), 1),
                            "samples": len(v)}
        return out or None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------


def _c2():
    from tests.gpu_cases import sigmoid_chain

    return sigmoid_chain(4096, 4096, seed=1)


def _c3():
    from tests.gpu_cases import softmax

    return softmax(8192, 8192, seed=2)


def _gemm():
    from tests.gpu_cases import plain_matmul

    return plain_matmul(4096, 4096, 4096, seed=0)


def _c4(diamond=False):
    from tests.gpu_cases import mlp_block

    return mlp_block(4096, 4096, 11008, seed=3, diamond=diamond)


def _c5(head=0):
    from tests.gpu_cases import attention_head

    return attention_head(2048, 128, seed=4, head=head, heads=32)


def _copy():
    """The shape-copy path (a reshape that cannot be a view): a transposed
    4096x4096 fp32 view flattened -- 64 MiB read, 64 MiB written."""
    from metellus_amd.orchestrator import Operations

    ops = Operations()
    ops.from_numpy(np.random.default_rng(5).standard_normal((4096, 4096)).astype(np.float32), "X")
    ops.transpose("X", out="Xt")
    ops.reshape("Xt", (4096 * 4096,), out="Y")
    return ops


# ---------------------------------------------------------------------------
# per-kernel algorithmic work
# ---------------------------------------------------------------------------


def kernel_work(group, tensors) -> tuple[str, float]:
    """('hbm', bytes) or ('mfma', flops) for one launch of ``group``:
    every binding read once plus the output written once (elementwise,
    reduction, copy); 2*M*N*K per anchor for matmul kernels."""
    from metellus_amd.orchestrator.ir import MatmulOp

    mm = [op for op in group.ops if isinstance(op, MatmulOp)]
    if mm:
        return "mfma", float(sum(2 * op.a.shape[0] * op.a.shape[1] * op.b.shape[1] for op in mm))
    nbytes = 0
    for key in group.bindings:
        nbytes += tensors[key].nbytes
    return "hbm", float(nbytes)


class Prepared:
    """A compiled program with device-resident inputs/outputs, ready for
    repeated timed launches of its kernels."""

    def __init__(self, ops):
        from metellus_amd.api import compile_program
        from metellus_amd.runtime import hip_backend
        from metellus_amd.runtime.buffer import Buffer

        self.ops = ops
        self.groups = compile_program(ops)
        self.tensors = ops.tensors
        self.env = {}
        nbytes = {op.out.buffer_key: op.out.nbytes for op in ops.build()}
        for name, arr in ops.uploads.items():
            self.env[name] = Buffer.from_numpy(arr)
        for g in self.groups:
            for k in g.bindings:
                if k not in self.env:
                    self.env[k] = Buffer(nbytes[k])
            _ = g.kernel.handle  # hiprtc compile outside the timed region
        self.hip = hip_backend
        # a key -> Tensor map for byte counts (owners)
        self.owner = {}
        for t in self.tensors.values():
            if t.buffer_key == t.name:
                self.owner[t.name] = t

    def launch(self, i, timed=False):
        g = self.groups[i]
        return self.hip.launch(
            g.kernel.handle, [self.env[k] for k in g.bindings], g.dims, g.kernel.dims_slot_index,
            g.grid, g.threads, timed=timed, workspace=g.kernel.workspace_bytes,
        )

    def run_all(self):
        for i in range(len(self.groups)):
            self.launch(i)

    def source_sha16(self, i: int) -> str:
        return source_sha16(self.groups[i].kernel.source)

    def download(self, key, shape):
        return self.env[key].numpy(shape, np.float32)

    def release(self):
        for b in self.env.values():
            b.release()
        self.env.clear()


class PreparedBatch:
    """Structurally identical programs (attention heads) with device-resident
    buffers and per-stage pointer tables, for timing batched launches."""

    def __init__(self, programs):
        from metellus_amd.api import compile_program
        from metellus_amd.runtime import hip_backend
        from metellus_amd.runtime.buffer import Buffer

        self.hip = hip_backend
        self.B = len(programs)
        self.programs = programs
        self.groups = compile_program(programs[0], batch=self.B)
        per = [compile_program(p, batch=self.B) for p in programs[1:]]
        for gs in per:
            assert [g.kernel.source for g in gs] == [g.kernel.source for g in self.groups]
        self.envs = []
        for ops in programs:
            env = {}
            nbytes = {op.out.buffer_key: op.out.nbytes for op in ops.build()}
            for name, arr in ops.uploads.items():
                env[name] = Buffer.from_numpy(arr)
            for g in self.groups:
                for k in g.bindings:
                    if k not in env:
                        env[k] = Buffer(nbytes[k])
            self.envs.append(env)
        self.tables = []
        for g in self.groups:
            tabs = [
                Buffer.from_numpy(np.array([env[k].device_address for env in self.envs], dtype=np.uint64))
                for k in g.bindings
            ]
            self.tables.append(tabs)
            _ = g.kernel.batched().handle
        self.owner = {t.name: t for t in programs[0].tensors.values() if t.buffer_key == t.name}

    def launch(self, i, timed=False):
        g = self.groups[i]
        k = g.kernel.batched()
        return self.hip.launch(
            k.handle, self.tables[i], g.dims, k.dims_slot_index,
            (g.grid[0], g.grid[1], g.grid[2] * self.B), g.threads, timed=timed, workspace=k.workspace_bytes,
        )

    def source_sha16(self, i: int) -> str:
        return source_sha16(self.groups[i].kernel.batched().source)

    def release(self):
        for env in self.envs:
            for b in env.values():
                b.release()
        for tabs in self.tables:
            for b in tabs:
                b.release()


class Flusher:
    """Evicts the 256 MiB Infinity Cache by *reading* a 512 MiB buffer (a
    row-sum kernel of this framework).  A write-based flush (memset) would
    leave dirty lines whose write-back then lands inside the measured
    kernel; after a read flush the cache holds only clean lines.  The flush
    kernel is built with ordinary (allocating) loads: nontemporal loads,
    the product default for row reductions, would leave the cache contents
    -- dirty output lines included -- in place."""

    ROWS, COLS = 16384, 8192  # 512 MiB of fp32

    def __init__(self):
        from metellus_amd.api import compile_program
        from metellus_amd.compute.reduction import reduction as red
        from metellus_amd.orchestrator import Operations
        from metellus_amd.runtime import hip_backend
        from metellus_amd.runtime.buffer import Buffer

        ops = Operations()
        ops.input("flush_src", (self.ROWS, self.COLS))
        ops.reduction("sum", out="flush_sum", x="flush_src")
        saved, red.NT_LOAD = red.NT_LOAD, False
        try:
            (self.group,) = compile_program(ops)
        finally:
            red.NT_LOAD = saved
        assert "mt_ld4_nt" not in self.group.kernel.source.split('extern "C"')[1]
        self.src = Buffer(self.ROWS * self.COLS * 4)
        self.src.fill(0)
        self.dst = Buffer(self.ROWS * 4)
        self.hip = hip_backend

    def flush(self):
        g = self.group
        self.hip.launch(g.kernel.handle, [self.src, self.dst], g.dims, g.kernel.dims_slot_index, g.grid, g.threads)

    def release(self):
        self.src.release()
        self.dst.release()


# Warm-up before a kernel's timed launches: at least WARM_MS of its own GPU
# time, run the way the timed launches are (flush, launch).  Measured on
# MI355X: the fp32 MFMA kernels start ~20 % slower (the clocks are still
# rising) and settle after ~15 ms of sustained work; with a 2-launch warm-up
# the attention S kernel read 351-374 us on its first launches and 293 us
# settled.  HBM-bound kernels run at their settled rate from the first launch.
WARM_MS = 50.0
WARM_MAX_LAUNCHES = 400


def warm_up(launch, flusher, min_launches: int = 2) -> int:
    """Flush + launch until ``WARM_MS`` of kernel time have run (and at
    least ``min_launches`` launches); returns the number of launches."""
    total, n = 0.0, 0
    while n < min_launches or (total < WARM_MS and n < WARM_MAX_LAUNCHES):
        if flusher is not None:
            flusher.flush()
        total += launch(True)
        n += 1
    return n


def time_kernels(prep: Prepared, steps: int, warmup: int, flusher, label: str) -> list[dict]:
    """Per kernel: warm up (``warm_up``), then ``steps`` event-timed
    launches, each after an Infinity Cache flush (when ``flusher`` is
    given)."""
    out = []
    for i, g in enumerate(prep.groups):
        warm_up(lambda timed, i=i: prep.launch(i, timed=timed), flusher, warmup)
        prep.hip.synchronize()
        ms = []
        sensors = GpuSensors()
        with sensors:
            for s in range(steps):
                if flusher is not None:
                    flusher.flush()
                ms.append(prep.launch(i, timed=True))
        prep.hip.check_workspace()  # raises if a stream-K launch gave up waiting
        bound, work = kernel_work(g, prep.owner)
        work *= getattr(prep, "B", 1)
        mean = float(np.mean(ms))
        if bound == "hbm":
            achieved = work / (mean * 1e-3) / 1e9
            peak, unit = HBM_PEAK_GBS, "GB/s"
        else:
            achieved = work / (mean * 1e-3) / 1e12
            peak, unit = FP32_MFMA_PEAK_TFLOPS, "TFLOP/s"
        out.append(
            {
                "kernel": g.kernel.function_name,
                "config": label,
                "source_sha16": prep.source_sha16(i),
                "strategy": g.strategy.value,
                "grid": list(g.grid),
                "threads": list(g.threads),
                "ms_mean": round(mean, 5),
                "ms_min": round(float(np.min(ms)), 5),
                "ms_median": round(float(np.median(ms)), 5),
                "bound": bound,
                "work": work,
                "achieved": round(achieved, 2),
                "peak": peak,
                "unit": unit,
                "frac": round(achieved / peak, 4),
                "sensors": sensors.summary(),
            }
        )
        log(f"[bench] {label} {g.kernel.function_name}: {mean:.4f} ms (median {np.median(ms):.4f})  "
            f"{achieved:.1f} {unit} ({100*achieved/peak:.1f}%)")
    return out


def check_c2(prep: Prepared) -> float:
    """Max abs error of the GPU output on 64 sampled rows against the chain
    sigmoid(a*b + c) * d in NumPy float32 (the whole-output checks against
    the oracle are GPU tests; this guards the timed run)."""
    out = prep.download("out", (4096, 4096))
    rows = np.random.default_rng(0).choice(4096, 64, replace=False)
    u = {k: prep.ops.uploads[k][rows] for k in "abcd"}
    one = np.float32(1.0)
    t = one / (np.exp(-(u["a"] * u["b"] + u["c"])) + one) * u["d"]
    err = np.abs(out[rows] - t)
    tol = 1e-5 + 1e-5 * np.abs(t)
    if not np.all(err <= tol):
        raise AssertionError(f"C2 output mismatch: max err {err.max():.3e}")
    return float(err.max())


def cpu_cores() -> int:
    """Host threads the CPU baselines use: the process's CPU affinity,
    capped by ``OMP_NUM_THREADS`` when set (the GPU boxes set it to the
    one-GPU share of the host)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def _split_rows(fn, pool, cores, *arrays):
    """``fn`` over row blocks of equally shaped arrays on ``pool`` (NumPy
    ufuncs release the GIL), results stacked in row order."""
    rows = arrays[0].shape[0]
    step = -(-rows // cores)
    parts = [pool.submit(fn, *(a[r : r + step] for a in arrays)) for r in range(0, rows, step)]
    return np.concatenate([p.result() for p in parts], axis=0)


def _numpy_program(label: str, made, pool, cores):
    """The configuration as one float32 expression over the oracle's op
    table (``oracle/ir_eval.apply_elementwise``), elementwise work split over
    row blocks on the thread pool, matmuls on NumPy's OpenBLAS sgemm."""
    from oracle.ir_eval import apply_elementwise as ew

    f32 = np.float32
    sig = lambda t: ew("recip", ew("add", ew("exp", ew("negate", t)), f32(1.0)))

    def softmax_block(x):
        m = np.max(x, axis=-1, keepdims=True)
        e = ew("exp", ew("subtract", x, m))
        return ew("div", e, np.sum(e, axis=-1, keepdims=True, dtype=f32))

    par = lambda fn, *a: _split_rows(fn, pool, cores, *a)
    if label.startswith("C2"):
        a, b, c, d = (made.uploads[k] for k in "abcd")
        return lambda: par(lambda a, b, c, d: ew("mul", sig(ew("add", ew("mul", a, b), c)), d), a, b, c, d)
    if label.startswith("C3"):
        x = made.uploads["x"]
        return lambda: par(softmax_block, x)
    if label.startswith("matmul"):
        a, b = made.uploads["A"], made.uploads["B"]
        return lambda: a @ b
    if label.startswith("C4"):
        u = made.uploads

        def once():
            h1, h2 = u["X"] @ u["W1"], u["X"] @ u["W2"]
            if "W3" not in u:  # the diamond variant stops at the product
                return par(lambda p, q: ew("mul", p, q), h1, h2)
            z = par(lambda p, q: ew("mul", ew("mul", p, sig(p)), q), h1, h2)
            return z @ u["W3"]

        return once
    if label.startswith("C5"):
        q, k, v = (np.stack([p.uploads[n] for p in made]) for n in "QKV")
        kt = k.transpose(0, 2, 1)
        scale = f32(1.0 / np.sqrt(q.shape[-1]))
        return lambda: par(lambda s: softmax_block(ew("mul", s, scale)), q @ kt) @ v
    return None


def _torch_program(label: str, made):
    """The same expression in torch on the CPU (float32, intra-op threads)."""
    import torch

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    if label.startswith("C2"):
        a, b, c, d = (t(made.uploads[k]) for k in "abcd")
        return lambda: torch.reciprocal(torch.exp(-(a * b + c)) + 1.0) * d
    if label.startswith("C3"):
        x = t(made.uploads["x"])

        def once():
            e = torch.exp(x - x.amax(dim=-1, keepdim=True))
            return e / e.sum(dim=-1, keepdim=True)

        return once
    if label.startswith("matmul"):
        a, b = t(made.uploads["A"]), t(made.uploads["B"])
        return lambda: a @ b
    if label.startswith("C4"):
        u = {k: t(v) for k, v in made.uploads.items()}

        def once():
            h1, h2 = u["X"] @ u["W1"], u["X"] @ u["W2"]
            if "W3" not in u:
                return h1 * h2
            return (h1 * torch.reciprocal(torch.exp(-h1) + 1.0) * h2) @ u["W3"]

        return once
    if label.startswith("C5"):
        q, k, v = (t(np.stack([p.uploads[n] for p in made])) for n in "QKV")
        kt = k.transpose(1, 2)
        scale = float(np.float32(1.0 / np.sqrt(q.shape[-1])))

        def once():
            s = (q @ kt) * scale
            e = torch.exp(s - s.amax(dim=-1, keepdim=True))
            return (e / e.sum(dim=-1, keepdim=True)) @ v

        return once
    return None


def _time_cpu(once, budget_s: float) -> tuple[float, int]:
    """Median seconds of ``once()`` over at least 3 runs after one warm-up,
    running for about ``budget_s``."""
    once()
    times, t0 = [], time.perf_counter()
    while len(times) < 3 or time.perf_counter() - t0 < budget_s:
        s = time.perf_counter()
        once()
        times.append(time.perf_counter() - s)
    return float(np.median(times)), len(times)


def cpu_baseline_config(label: str, made, per_kernel: list[dict], budget_s: float = 3.0) -> dict | None:
    """Time one whole configuration on the host CPU in float32, on
    ``cpu_cores()`` threads: the oracle-op-table NumPy expression (OpenBLAS
    and the elementwise thread pool both pinned to that count) and, beside
    it, torch on the CPU (``torch.set_num_threads`` to the same count).
    Throughput uses the configuration's algorithmic work: the matmul flops
    when it has matmuls, else the kernels' algorithmic bytes."""
    from concurrent.futures import ThreadPoolExecutor

    import threadpoolctl
    import torch

    cores = cpu_cores()
    mine = [k for k in per_kernel if k["config"] == label]
    if not mine:
        return None
    if any(k["bound"] == "mfma" for k in mine):
        work, unit, div = sum(k["work"] for k in mine if k["bound"] == "mfma"), "TFLOP/s", 1e12
    else:
        work, unit, div = sum(k["work"] for k in mine), "GB/s", 1e9
    with ThreadPoolExecutor(cores) as pool, threadpoolctl.threadpool_limits(cores):
        once = _numpy_program(label, made, pool, cores)
        if once is None:
            return None
        med, n = _time_cpu(once, budget_s)
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        tmed, tn = _time_cpu(_torch_program(label, made), budget_s)
    finally:
        torch.set_num_threads(prev)
    gpu_ms = sum(k["ms_mean"] for k in mine)
    return {
        "config": label,
        "value": round(work / med / div, 4),
        "unit": unit,
        "cores": cores,
        "kind": "port",
        "sample": f"whole configuration on the full inputs, float32: oracle op table over NumPy "
        f"(OpenBLAS sgemm and a {cores}-thread elementwise pool), {n} evaluations, median {med * 1e3:.1f} ms",
        "ms": round(med * 1e3, 3),
        "torch_cpu": {
            "value": round(work / tmed / div, 4),
            "unit": unit,
            "cores": cores,
            "ms": round(tmed * 1e3, 3),
            "sample": f"torch {torch.__version__} CPU float32, {cores} intra-op threads, {tn} evaluations",
        },
        "gpu_kernels_ms": round(gpu_ms, 4),
        "gpu_over_cpu": round(min(med, tmed) * 1e3 / gpu_ms, 1) if gpu_ms > 0 else None,
    }


def end_to_end_runs(reps: int = 5) -> list[dict]:
    """``api.run`` wall time (compile lookup, uploads from NumPy, kernels,
    download of the final output) for C2 and C3 -- the reference API's
    whole path, host transfers included; never part of ``value``."""
    from metellus_amd.api import run

    out = []
    for label, make, outputs in (("C2", _c2, ("out",)), ("C3 softmax", _c3, ("p",))):
        ops = make()
        run(ops, outputs=outputs)  # compile, pools and staging buffers warm
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            run(ops, outputs=outputs)
            ts.append(time.perf_counter() - t0)
        up = sum(a.nbytes for a in ops.uploads.values())
        out.append({"config": label, "run_ms_median": round(float(np.median(ts)) * 1e3, 3),
                    "run_ms_min": round(min(ts) * 1e3, 3), "uploaded_bytes": up, "downloaded": list(outputs)})
        log(f"[bench] run() {label}: median {np.median(ts) * 1e3:.2f} ms ({up / 2**20:.0f} MiB uploaded)")
    return out


def ceiling_benches(steps: int, flusher) -> list[dict]:
    """HBM ceilings of C2's access pattern through this framework's own
    kernels with trivial arithmetic: 4 reads + 1 write of 64 MiB each (C2's
    bytes, adds instead of the sigmoid chain), 1 read + 1 write (a copy),
    and reads only (a row sum of 256 MiB).  C2 at the 4-read-1-write figure
    means its chain costs nothing and the kernel is at the pattern's HBM
    limit on this box."""
    from metellus_amd.orchestrator import Operations

    rng = np.random.default_rng(7)
    mk = lambda shape: rng.standard_normal(shape).astype(np.float32)
    out = []
    ops = Operations()
    for n in "abcd":
        ops.from_numpy(mk((4096, 4096)), n)
    ops.elementwise("add", out="t1", operands=("a", "b"))
    ops.elementwise("add", out="t2", operands=("t1", "c"))
    ops.elementwise("add", out="sum4", operands=("t2", "d"))
    cases = [("ceiling: 4 reads + 1 write, 64 MiB each", ops)]
    ops = Operations()
    ops.from_numpy(mk((4096, 4096)), "x")
    ops.elementwise("mul", out="copy", operands=("x", 1.0))
    cases.append(("ceiling: 1 read + 1 write, 64 MiB each", ops))
    ops = Operations()
    ops.from_numpy(mk((8192, 8192)), "x")
    ops.reduction("sum", out="rows", x="x")
    cases.append(("ceiling: read 256 MiB (row sums)", ops))
    for label, ops in cases:
        prep = Prepared(ops)
        out += time_kernels(prep, steps, 2, flusher, label)
        prep.release()
    return out


# A read-only stream of a different design from the framework's row
# reductions (one wave per row): workgroup g reads the g-th contiguous
# chunk of n / grid float4s, its lanes on adjacent 16-byte slots with four
# 128-bit nontemporal loads in flight each, then each wave writes one
# partial sum.  Its time is a ceiling for reads on the box that does not
# depend on the generated kernels (the best of the designs measured:
# grid-stride walks with 4-16 loads in flight ran at 5.3-6.8 TB/s).
READ_CEILING_SRC = r"""
typedef float rc_f4 __attribute__((ext_vector_type(4)));
struct rc_dims { unsigned int v[16]; };
extern "C" __global__ void __launch_bounds__(256)
read_ceiling(const rc_f4* __restrict__ x, float* __restrict__ out, const rc_dims dims) {
    const unsigned per = dims.v[0] / gridDim.x;
    const rc_f4* p = x + (size_t)blockIdx.x * per;
    rc_f4 a = {0.f, 0.f, 0.f, 0.f}, b = a, c = a, d = a;
    unsigned j = threadIdx.x;
    for (; j + 768u < per; j += 1024u) {
        a += __builtin_nontemporal_load(p + j);
        b += __builtin_nontemporal_load(p + j + 256u);
        c += __builtin_nontemporal_load(p + j + 512u);
        d += __builtin_nontemporal_load(p + j + 768u);
    }
    for (; j < per; j += 256u) a += __builtin_nontemporal_load(p + j);
    a += b + c + d;
    float s = (a.x + a.y) + (a.z + a.w);
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63u) == 0u) out[blockIdx.x * 4u + (threadIdx.x >> 6)] = s;
}
"""
READ_CEILING_GRIDS = (2048, 8192, 32768)  # workgroups of 256 lanes; each divides the float4 count
SWEEP_SCALES = (1, 2, 4)


def read_ceiling(buf, nbytes: int, steps: int, flusher, label: str) -> list[dict]:
    """Time ``read_ceiling`` over the first ``nbytes`` of ``buf`` at each of
    ``READ_CEILING_GRIDS``; work = bytes read + the partial sums written."""
    from metellus_amd.runtime import hip_backend
    from metellus_amd.runtime.buffer import Buffer

    n4 = nbytes // 16
    if nbytes % 16 or n4 >= 2**32 or nbytes > buf.nbytes or any(n4 % g for g in READ_CEILING_GRIDS):
        raise ValueError(f"read_ceiling: {nbytes} bytes do not split into the kernel's float4 chunks or fit the buffer")
    kernel = hip_backend.compile_kernel(READ_CEILING_SRC, "read_ceiling")
    out = Buffer(4 * 4 * max(READ_CEILING_GRIDS))
    recs = []
    for grid in READ_CEILING_GRIDS:
        def launch(timed, grid=grid):
            return hip_backend.launch(kernel, [buf, out], [nbytes // 16], 2, (grid, 1, 1), (256, 1, 1), timed=timed)
        warm_up(launch, flusher, 2)
        hip_backend.synchronize()
        ms = []
        for _ in range(steps):
            if flusher is not None:
                flusher.flush()
            ms.append(launch(True))
        work = float(nbytes + 4 * 4 * grid)
        mean = float(np.mean(ms))
        achieved = work / (mean * 1e-3) / 1e9
        recs.append({"kernel": "read_ceiling", "config": f"{label} grid {grid}", "grid": [grid, 1, 1],
                     "threads": [256, 1, 1], "ms_mean": round(mean, 5), "ms_min": round(float(np.min(ms)), 5),
                     "ms_median": round(float(np.median(ms)), 5), "bound": "hbm", "work": work,
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4)})
        log(f"[bench] {label} read_ceiling grid {grid}: {mean:.4f} ms  {achieved:.1f} GB/s "
            f"({100 * achieved / HBM_PEAK_GBS:.1f}%)")
    out.release()
    return recs


def fit_sweep(records: list[dict]) -> list[dict]:
    """Least-squares ``t = t0 + bytes / rate`` per kernel over the sweep's
    sizes: ``rate`` is the steady-state stream rate, ``t0`` the fixed cost
    (launch ramp, tail) that the smaller sizes cannot amortise."""
    groups: dict[str, list[tuple[float, float]]] = {}
    for r in records:
        fam = r["config"].split(" x", 1)[0] + " / " + r["kernel"] + (
            " " + r["config"].rsplit(" ", 2)[-2] + " " + r["config"].rsplit(" ", 1)[-1]
            if r["kernel"] == "read_ceiling" else "")
        groups.setdefault(fam, []).append((r["work"], r["ms_mean"] * 1e-3))
    fits = []
    for fam, pts in groups.items():
        if len(pts) < 2:
            continue
        x = np.array([p[0] for p in pts])
        t = np.array([p[1] for p in pts])
        b, a = np.polyfit(x, t, 1)
        fits.append({"family": fam, "sizes_bytes": [int(v) for v in x], "steady_GBps": round(1 / b / 1e9, 1),
                     "steady_frac": round(1 / b / 1e9 / HBM_PEAK_GBS, 4), "fixed_us": round(a * 1e6, 2),
                     "frac_per_size": [round(v / s / 1e9 / HBM_PEAK_GBS, 4) for v, s in zip(x, t)]})
        log(f"[bench] sweep fit {fam}: steady {1 / b / 1e9:.0f} GB/s ({100 / b / 1e9 / HBM_PEAK_GBS:.1f}%), "
            f"fixed {a * 1e6:.2f} us")
    return fits


def hbm_sweep(steps: int, flusher) -> tuple[list[dict], list[dict]]:
    """C2 (4 reads + 1 write) and C3 (row reductions and broadcast tiled
    streams) at 1x, 2x and 4x their BASELINE sizes, plus ``read_ceiling``
    over C3's input, each launch after the cache flush.  Returns the
    per-kernel records and the ``fit_sweep`` lines."""
    from tests.gpu_cases import sigmoid_chain, softmax

    recs = []
    for s in SWEEP_SCALES:
        for label, ops in ((f"sweep C2 x{s}", sigmoid_chain(4096 * s, 4096, seed=1)),
                           (f"sweep C3 x{s}", softmax(8192 * s, 8192, seed=2))):
            log(f"[bench] {label}: preparing")
            prep = Prepared(ops)
            recs += time_kernels(prep, steps, 2, flusher, label)
            if label.startswith("sweep C3"):
                recs += read_ceiling(prep.env["x"], 8192 * s * 8192 * 4, steps, flusher, f"sweep read x{s}")
            prep.release()
            del ops
    return recs, fit_sweep(recs)


def fragment_benches(steps: int, flusher) -> list[dict]:
    """The reference's fragment-level benches (tests/bench_init.py,
    bench_reduction.py, bench_elementwise.py, bench_matmul.py) at their own
    sizes, composed by hand as in ``tests/fragment_kernels.py``; each launch
    timed after a cache flush.  Work: bytes read + written once, or 2*M*N*K."""
    import metellus_amd

    metellus_amd.install_reference_namespace()  # the builders import the reference's module names
    from metellus_amd.compute.elementwise.elementwise import elementwise_arity
    from metellus_amd.runtime import hip_backend
    from metellus_amd.runtime.buffer import Buffer
    from tests import fragment_kernels as fk

    rng = np.random.default_rng(17)
    out = []

    def time_one(label, kernel, arrays, out_bytes, dims, grid, threads, work, bound):
        bufs = [Buffer.from_numpy(a) if isinstance(a, np.ndarray) else Buffer(a) for a in arrays]
        handle = kernel.handle

        def launch(timed):
            return hip_backend.launch(handle, bufs, dims, kernel.dims_slot_index, grid, threads, timed=timed)

        warm_up(launch, flusher)
        ms = []
        for s in range(steps):
            if flusher is not None:
                flusher.flush()
            ms.append(launch(True))
        for b in bufs:
            b.release()
        mean = float(np.mean(ms))
        if bound == "hbm":
            achieved, peak, unit = work / (mean * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        else:
            achieved, peak, unit = work / (mean * 1e-3) / 1e12, FP32_MFMA_PEAK_TFLOPS, "TFLOP/s"
        log(f"[bench] {label}: {mean:.4f} ms  {achieved:.1f} {unit} ({100 * achieved / peak:.1f}%)")
        out.append({"kernel": kernel.function_name, "config": label, "grid": list(grid), "threads": list(threads),
                    "ms_mean": round(mean, 5), "ms_min": round(float(np.min(ms)), 5), "bound": bound,
                    "work": float(work), "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                    "frac": round(achieved / peak, 4)})

    n = 1 << 22  # 4M floats, bench_init's size
    tg = (fk.TG_X, 1, 1)
    time_one("bench_init fill 4M", fk.fill_kernel(1.0), [n * 4], 0, (n,), fk.init_grid(n), tg, n * 4, "hbm")
    time_one("bench_init arange 4M", fk.arange_kernel(0.0, 1.0), [n * 4], 0, (n,), fk.init_grid(n), tg, n * 4, "hbm")
    src = rng.standard_normal(n).astype(np.float32)
    time_one("bench_init copy 4M", fk.copy_kernel(), [n * 4, src], 0, (n,), fk.init_grid(n), tg, 2 * n * 4, "hbm")

    m = k = 1024  # bench_reduction's and bench_elementwise's size
    x = rng.uniform(-1.0, 1.0, (m, k)).astype(np.float32)
    for op in ("sum", "max", "min", "product"):
        time_one(f"bench_reduction {op} 1024x1024", fk.reduction_kernel(op), [x, m * 4], 0, (m, k), (m, 1, 1), tg,
                 x.nbytes + m * 4, "hbm")

    xe = rng.uniform(0.25, 3.75, (m, k)).astype(np.float32)
    ye = rng.uniform(1.25, 2.25, (m, k)).astype(np.float32)
    cases = [(op, None, None, "none") for op in ("negate", "exp", "sqrt", "tanh")]
    cases += [(op, ye, None, "none") for op in ("add", "mul", "div", "max", "lt")]
    cases += [("add", np.array([[1.5]], np.float32), None, "scalar"),
              ("add", rng.uniform(0.5, 1.5, (1, k)).astype(np.float32), None, "row"),
              ("mul", rng.uniform(0.5, 1.5, (m, 1)).astype(np.float32), None, "col"),
              ("where", ye, (xe > 2.0).astype(np.float32), "none")]
    for op, y, cond, yb in cases:
        kernel, bindings, dims, grid, threads = fk.elementwise_kernel(
            op, m, k, y.shape if y is not None else None, cond.shape if cond is not None else None, yb, "none")
        arrays = [xe] + ([y] if y is not None else []) + ([cond] if cond is not None else []) + [m * k * 4]
        work = sum(a.nbytes for a in arrays[:-1]) + m * k * 4
        assert elementwise_arity(op) == len(arrays) - 1
        time_one(f"bench_elementwise {op} ({yb}) 1024x1024", kernel, arrays, 0, dims, grid, threads, work, "hbm")

    # the same kernels at a size where bandwidth, not launch latency, decides
    big = 1 << 26  # 64M floats = 256 MiB
    time_one("bench_init fill 64M (scale)", fk.fill_kernel(1.0), [big * 4], 0, (big,), fk.init_grid(big), tg,
             big * 4, "hbm")
    bsrc = rng.standard_normal(big).astype(np.float32)
    time_one("bench_init copy 64M (scale)", fk.copy_kernel(), [big * 4, bsrc], 0, (big,), fk.init_grid(big), tg,
             2 * big * 4, "hbm")
    del bsrc
    xb = rng.standard_normal((8192, 8192)).astype(np.float32)
    time_one("bench_reduction sum 8192x8192 (scale)", fk.reduction_kernel("sum"), [xb, 8192 * 4], 0, (8192, 8192),
             (8192, 1, 1), tg, xb.nbytes + 8192 * 4, "hbm")
    kernel, bindings, dims, grid, threads = fk.elementwise_kernel("add", 8192, 8192, (8192, 8192), None, "none", "none")
    time_one("bench_elementwise add 8192x8192 (scale)", kernel, [xb, xb, 8192 * 8192 * 4], 0, dims, grid, threads,
             3 * xb.nbytes, "hbm")
    del xb

    for mm, kk, nn in ((512, 512, 512), (1024, 64, 1024), (4096, 512, 4096), (8192, 64, 8192)):
        a = rng.standard_normal((mm, kk)).astype(np.float32)
        b = rng.standard_normal((kk, nn)).astype(np.float32)
        kernel, tile, aligned, grid = fk.gemm_kernel(mm, kk, nn)
        time_one(f"bench_matmul {mm}x{kk}x{nn}", kernel, [a, b, mm * nn * 4], 0, (mm, kk, nn), grid,
                 (tile.tg_x, tile.tg_y, 1), 2.0 * mm * kk * nn, "mfma")
    return out


PMC_PROFILE = "bench_kernels_pmc.txt"


def read_profile_traffic(config: str, kernel: str, sha16: str, name: str = PMC_PROFILE) -> dict:
    """HBM bytes per launch of ``kernel`` in ``config`` from the committed
    rocprofv3 PMC summary: its table row ``config  kernel  source-sha16
    algorithmic read written ...`` (FETCH_SIZE and WRITE_SIZE, copy-kernel
    calibrated), read + written.  The figure is used only when the row's
    source hash is ``sha16``, the hash of the kernel this run launches: a
    profile of an older version of the kernel gives ``traffic`` None and
    says so."""
    import re

    path = os.path.join(ROOT, "profiles", name)
    src = {"file": f"profiles/{name}", "kernel_source_sha16": sha16, "profiled_source_sha16": None,
           "matches": False}
    if not os.path.exists(path):
        return {"traffic": None, "source": src}
    pat = re.compile(r"^(.+?)\s{2,}(\S+)\s+([0-9a-f]{16})\s+(\(mfma\)|\d+)\s+(\d+)\s+(\d+)")
    with open(path, encoding="utf-8") as f:
        for line in f:
            m = pat.match(line)
            if m and m.group(1).strip() == config[:32].strip() and m.group(2) == kernel:
                src["profiled_source_sha16"] = m.group(3)
                src["matches"] = m.group(3) == sha16
                traffic = float(int(m.group(5)) + int(m.group(6))) if src["matches"] else None
                return {"traffic": traffic, "source": src}
    return {"traffic": None, "source": src}


C4_LABEL = "C4 MLP literal"
# The same C4 program with the multi-anchor merge-chain extension
# (orchestrator.fusion.MULTI_ANCHOR_MERGE_CHAINS): the gate in one kernel.
C4_EXT_LABEL = "C4 MLP literal, gate fused (extension)"
# C5 with the matmul -> reduction epilogue extension
# (orchestrator.fusion.MATMUL_REDUCTION_EPILOGUES): m1 = max(S) in S's kernel.
C5_EXT_LABEL = "C5 attention, row max fused (extension)"
EXTENSION_FLAGS = {C4_EXT_LABEL: "MULTI_ANCHOR_MERGE_CHAINS", C5_EXT_LABEL: "MATMUL_REDUCTION_EPILOGUES"}
C4_FLOPS = 3 * 2 * 4096 * 4096 * 11008  # 1.108 TFLOP of matmul work per step


def check_c4(prep: Prepared, rows: int = 64) -> float:
    """Sampled rows of the C4 output against float64 from the GPU's own
    ``z = h1 * s * h2`` (the W3 kernel's A operand): the whole-output checks
    are GPU tests; this guards the timed run.  Returns the max abs error."""
    from tests.matmul_check import check_matmul

    pick = np.sort(np.random.default_rng(0).choice(4096, rows, replace=False))
    h1, s, h2, out = (prep.download(k, (4096, 11008) if k != "out" else (4096, 4096)) for k in ("h1", "s", "h2", "out"))
    z = (h1[pick] * s[pick]) * h2[pick]
    w3 = prep.ops.uploads["W3"]
    check_matmul(out[pick], z, w3, "C4 out (sampled rows)")
    return float(np.abs(out[pick].astype(np.float64) - z.astype(np.float64) @ w3.astype(np.float64)).max())


def headline_c4(args, flush, info) -> tuple[dict, dict]:
    """Time ``args.steps`` C4 steps (flush, then the 4 kernels back to back
    between stream markers).  Returns the JSON line and the per-kernel
    records of the in-step kernel times."""
    from metellus_amd.runtime import hip_backend

    prep = Prepared(_c4(False))
    n = len(prep.groups)
    assert n == 4 and n + 1 <= 16, [g.kernel.function_name for g in prep.groups]
    for i in range(n):
        warm_up(lambda timed, i=i: prep.launch(i, timed=timed), flush, args.warmup)
    hip_backend.synchronize()
    step_ms, kern_ms = [], [[] for _ in range(n)]
    sensors = GpuSensors()
    with sensors:
        t0 = time.perf_counter()
        for _ in range(args.steps):
            if flush is not None:
                flush.flush()
            hip_backend.mark(0)
            for i in range(n):
                prep.launch(i)
                hip_backend.mark(i + 1)
            step_ms.append(hip_backend.mark_elapsed(0, n))
            for i in range(n):
                kern_ms[i].append(hip_backend.mark_elapsed(i, i + 1))
        hip_backend.synchronize()
        wall = time.perf_counter() - t0
    hip_backend.check_workspace()
    err = check_c4(prep)
    ms = float(np.mean(step_ms))
    tflops = C4_FLOPS / (ms * 1e-3) / 1e12
    records = []
    for i, g in enumerate(prep.groups):
        bound, work = kernel_work(g, prep.owner)
        mean = float(np.mean(kern_ms[i]))
        if bound == "hbm":
            achieved, peak, unit = work / (mean * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        else:
            achieved, peak, unit = work / (mean * 1e-3) / 1e12, FP32_MFMA_PEAK_TFLOPS, "TFLOP/s"
        records.append({
            "kernel": g.kernel.function_name, "config": C4_LABEL + " (in-step)",
            "source_sha16": prep.source_sha16(i), "strategy": g.strategy.value,
            "grid": list(g.grid), "threads": list(g.threads), "ms_mean": round(mean, 5),
            "ms_min": round(float(np.min(kern_ms[i])), 5), "ms_median": round(float(np.median(kern_ms[i])), 5),
            "bound": bound, "work": work, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4),
        })
    dom = max(records, key=lambda r: r["ms_mean"])
    traffic = read_profile_traffic(C4_LABEL, dom["kernel"], dom["source_sha16"])
    line = {
        "metric": "fused-kernel fp32 TFLOP/s & HBM GB/s (% of roofline), 1×MI355X",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0, 1/sqrt(fan_in)), numpy seed 3)",
        "config": {
            "workload": "C4: out = (silu(X@W1) * (X@W2)) @ W3, X 4096x4096, W1/W2 4096x11008, W3 11008x4096 fp32 "
            "(BASELINE.json configs[3], the largest configuration); 4 fused kernels per step",
            "kernels": [g.kernel.function_name for g in prep.groups],
            "flops_per_step": C4_FLOPS,
            "step_ms_min": round(float(np.min(step_ms)), 5),
            "step_ms_median": round(float(np.median(step_ms)), 5),
            "fraction_of_fp32_mfma_peak": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4),
            "cache_flush_between_steps": flush is not None,
            "wall_ms_per_step_incl_flush": round(wall * 1e3 / args.steps, 4),
            "max_abs_err_vs_float64_sampled_rows": err,
            "device": info["arch"],
            # which GPU the line ran on, and its clocks / power while the
            # timed steps ran (sampled every ~1 ms; None where unreadable)
            "device_identity": {k: info[k] for k in ("pci_bus_id", "memory_clock_khz", "memory_bytes", "host")},
            "sensors_during_steps": sensors.summary(),
            "sensors_scope": "every ~1 ms over the timed steps (back to back); per_kernel sensors span each "
                             "kernel's timing loop, flushes and host waits included",
            "parallelism": "1 GPU",
        },
        "roofline": {
            "kernel": dom["kernel"],
            "bound": dom["bound"],
            "achieved": dom["achieved"],
            "peak": dom["peak"],
            "unit": dom["unit"],
            "frac": dom["frac"],
            "traffic": traffic["traffic"],
            "traffic_source": traffic["source"],
        },
    }
    log(f"[bench] C4: {ms:.4f} ms/step, {tflops:.2f} TFLOP/s ({100 * tflops / FP32_MFMA_PEAK_TFLOPS:.1f}% of "
        f"fp32 MFMA peak); dominant {dom['kernel']} {dom['ms_mean']:.4f} ms ({100 * dom['frac']:.1f}%)")
    for r in records:
        log(f"[bench]   {r['kernel']}: {r['ms_mean']:.4f} ms  {r['achieved']:.1f} {r['unit']} ({100 * r['frac']:.1f}%)")
    made = prep.ops
    prep.release()
    return line, {"records": records, "made": made}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--only", default=None)
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-flush", action="store_true")
    ap.add_argument(
        "--calibrate-copy",
        action="store_true",
        help="also launch a plain 64 MiB -> 64 MiB copy kernel (for scaling PMC byte counters)",
    )
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py: this build measures one MI355X; the path shards by rows / heads / output "
            "tiles with no exchange, and multi-GPU runs are not part of it. "
            f"Requested --gpus {args.gpus} (WORLD_SIZE={world}).",
            file=sys.stderr,
        )
        return 2

    from metellus_amd.runtime import hip_backend
    info = {**hip_backend.device_info(), **hip_backend.device_pci(), "host": os.uname().nodename}
    GpuSensors.PCI_BUS_ID = info["pci_bus_id"]
    log(f"[bench] device {info}")
    flush = None if args.no_flush else Flusher()

    # ---- headline: C4 literal ----------------------------------------------
    only = args.only
    line = None
    per_config: list[dict] = []
    cpu_configs: list[dict] = []
    if only in (None, "c4"):
        log("[bench] C4 MLP block (headline): preparing")
        line, head = headline_c4(args, flush, info)
        per_config += head["records"]
        if not args.no_cpu:
            log(f"[bench] C4 CPU baseline on {cpu_cores()} threads (~20 s)")
            cpu = cpu_baseline_config(C4_LABEL + " (in-step)", head["made"], per_config, budget_s=10.0)
            cpu["config"] = C4_LABEL
            line["cpu_baseline"] = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample", "ms", "torch_cpu")}
            log(f"[bench] C4 CPU: {cpu['value']} TFLOP/s oracle/NumPy, {cpu['torch_cpu']['value']} TFLOP/s torch "
                f"on {cpu['cores']} threads")
        del head

    if args.calibrate_copy:
        log("[bench] copy calibration: 64 MiB in, 64 MiB out")
        from metellus_amd.orchestrator import Operations

        ops = Operations()
        ops.from_numpy(np.random.default_rng(0).standard_normal((4096, 4096)).astype(np.float32), "cx")
        ops.elementwise("mul", out="copyout", operands=("cx", 1.0))
        prep = Prepared(ops)
        per_config += time_kernels(prep, args.steps, 2, flush, "copy calibration 64 MiB")
        prep.release()

    if only == "fragments":
        per_config += fragment_benches(max(3, min(args.steps, 10)), flush)
    if only == "ceilings":
        per_config += ceiling_benches(max(3, args.steps), flush)
    sweep_fits = None
    if only == "sweep":
        recs, sweep_fits = hbm_sweep(max(3, args.steps), flush)
        per_config += recs

    # ---- other configs -----------------------------------------------------
    if (not args.no_extra and only is None) or only not in (None, "fragments"):
        extra_steps = max(3, args.steps)
        todo = []
        if only in (None, "c2"):
            todo.append(("C2 sigmoid chain 4096x4096", _c2))
        if only in (None, "c3"):
            todo.append(("C3 softmax 8192x8192", _c3))
        if only in (None, "gemm"):
            todo.append(("matmul 4096^3", _gemm))
        if only in (None, "c4"):
            todo.append(("C4 MLP literal", lambda: _c4(False)))
            todo.append(("C4 MLP diamond", lambda: _c4(True)))
            todo.append((C4_EXT_LABEL, lambda: _c4(False)))
        if only in (None, "c5"):
            todo.append(("C5 attention, 32 heads batched", lambda: [_c5(h) for h in range(32)]))
            todo.append((C5_EXT_LABEL, lambda: [_c5(h) for h in range(32)]))
        if only in (None, "copy"):
            todo.append(("shape copy: transposed 4096x4096 view", _copy))
        for label, make in todo:
            log(f"[bench] {label}: preparing")
            made = make()
            from metellus_amd.orchestrator import fusion

            saved = {f: getattr(fusion, f) for f in EXTENSION_FLAGS.values()}
            for f in saved:
                setattr(fusion, f, EXTENSION_FLAGS.get(label) == f)
            try:
                prep = PreparedBatch(made) if isinstance(made, list) else Prepared(made)
            finally:
                for f, v in saved.items():
                    setattr(fusion, f, v)
            per_config += time_kernels(prep, extra_steps, 2, flush, label)
            if label.startswith("C2"):
                check_c2(prep)
            prep.release()
            if label in EXTENSION_FLAGS:  # the same program as its reference line: its CPU time is that line's
                continue
            if not args.no_cpu and not (label == C4_LABEL and line is not None):  # the headline timed C4 already
                cpu = cpu_baseline_config(label, made, per_config)
                if cpu is not None:
                    cpu_configs.append(cpu)
                    log(f"[bench] {label} CPU: {cpu['value']} {cpu['unit']} on {cpu['cores']} threads "
                        f"({cpu['ms']:.1f} ms; GPU kernels {cpu['gpu_kernels_ms']:.3f} ms)")
    if line is None:
        line = {"metric": "fused-kernel fp32 TFLOP/s & HBM GB/s (% of roofline), 1×MI355X", "value": None}
    if cpu_configs:
        line.setdefault("cpu_baseline", {})["per_config"] = cpu_configs
    line["per_kernel"] = per_config
    if sweep_fits is not None:
        line["hbm_sweep"] = sweep_fits
    if only is None and not args.no_extra:
        line["end_to_end"] = end_to_end_runs()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
