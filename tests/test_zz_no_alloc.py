"""The allocation-free launch (``mt_launch_noalloc``) through the C ABI,
against ``mt_launch`` with the shim's allocated workspace: stream-K matmul
kernels (the kernels that use a scratch buffer) give bit-identical outputs
from both entry points, on consecutive calls that shrink -- C4's X @ W1 at
its full size with the real resident capacity (the whole 64 MiB of partial
tiles), then smaller forced-capacity matmuls and a diamond with two
accumulator sets, whose calls reuse the same scratch; and the matmul ->
reduction epilogue extension in its workspace form (row-block counters in
the scratch's flag words).  The scratch error word stays 0, and a request
beyond the scratch's size is refused before anything is launched.  Around
every allocation-free call the shim's allocation counters, its live buffers
and its workspace size stay as they were; in a fresh process the call runs
before any workspace exists and leaves none behind."""

from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

from metellus_amd.api import compile_program
from metellus_amd.compute.matmul import config
from metellus_amd.orchestrator import Operations
from metellus_amd.runtime import hip_backend
from metellus_amd.runtime.buffer import Buffer
from tests import gpu_cases

pytestmark = pytest.mark.gpu

SCRATCH_MAX = 4096 + (64 << 20)


def _both(ops, out_name: str):
    """Outputs of the program's single stream-K kernel from mt_launch (with
    the shim workspace) and from mt_launch_noalloc (static scratch)."""
    (g,) = compile_program(ops)
    ws = g.kernel.workspace_bytes
    assert ws > 0, "the case must compile to a stream-K kernel"
    assert ws <= SCRATCH_MAX
    inputs = {k: Buffer.from_numpy(a) for k, a in ops.uploads.items()}
    shape = ops.tensors[out_name].shape
    nbytes = int(np.prod(shape)) * 4
    outs = []
    for noalloc in (False, True):
        out = Buffer(nbytes)
        out.fill(0xFF)  # NaN pattern: every element must be written
        bufs = [inputs[k] if k in inputs else out for k in g.bindings]
        args = (g.kernel.handle, bufs, g.dims, g.kernel.dims_slot_index, g.grid, g.threads)
        if noalloc:
            _noalloc_call(args, ws)
        else:
            hip_backend.launch(*args, workspace=ws)
            hip_backend.check_workspace()
        outs.append(out.numpy(shape, np.float32))
        out.release()
    for b in inputs.values():
        b.release()
    return outs


def _noalloc_call(args, ws: int) -> None:
    """One mt_launch_noalloc call (waited for) that must allocate nothing:
    the shim's device and host allocation counts, its live buffers and its
    workspace size are the same before and after it."""
    before = hip_backend.alloc_stats()
    assert hip_backend.launch_noalloc(*args, scratch=ws) == 0
    assert hip_backend.alloc_stats() == before


def _forced(monkeypatch, capacity):
    monkeypatch.setattr(config, "PERSISTENT", True)
    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", capacity)
    monkeypatch.setattr(config, "STREAM_K", True)


def test_noalloc_matches_mt_launch_on_shrinking_calls(monkeypatch):
    hip_backend.init()
    print("noalloc: C4 X@W1 4096x4096x11008, real capacity", flush=True)
    big = gpu_cases.mlp_block(4096, 4096, 11008, seed=3, diamond=False)
    ops = Operations()
    ops.from_numpy(big.uploads["X"], "X")
    ops.from_numpy(big.uploads["W1"], "W1")
    ops.matmul(a="X", b="W1", out="h1")
    a, b = _both(ops, "h1")
    assert not np.isnan(a).any()
    np.testing.assert_array_equal(a, b)
    del big, ops, a, b

    for (M, K, N), cap in (((1024, 256, 1024), 5), ((640, 128, 768), 7)):
        print(f"noalloc: plain matmul {(M, K, N)} capacity {cap}", flush=True)
        _forced(monkeypatch, cap)
        a, b = _both(gpu_cases.plain_matmul(M, K, N, seed=31), "C")
        assert not np.isnan(a).any()
        np.testing.assert_array_equal(a, b)

    print("noalloc: diamond 512x256x640 capacity 6", flush=True)
    _forced(monkeypatch, 6)
    a, b = _both(gpu_cases.mlp_block(512, 256, 640, seed=32, diamond=True), "z")
    assert not np.isnan(a).any()
    np.testing.assert_array_equal(a, b)


def test_noalloc_refuses_oversized_scratch(monkeypatch):
    hip_backend.init()
    _forced(monkeypatch, 5)
    ops = gpu_cases.plain_matmul(1024, 256, 1024, seed=33)
    (g,) = compile_program(ops)
    inputs = {k: Buffer.from_numpy(a) for k, a in ops.uploads.items()}
    out = Buffer(1024 * 1024 * 4)
    bufs = [inputs[k] if k in inputs else out for k in g.bindings]
    with pytest.raises(RuntimeError, match="static scratch holds"):
        hip_backend.launch_noalloc(g.kernel.handle, bufs, g.dims, g.kernel.dims_slot_index, g.grid, g.threads,
                                   scratch=SCRATCH_MAX + 4)


def _row_max_program(M: int, K: int, N: int, seed: int) -> Operations:
    rng = np.random.default_rng(seed)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    ops.matmul(a="A", b="B", out="Y")
    ops.elementwise("mul", out="Yc", operands=("Y", 0.5))
    ops.reduction("max", out="r", x="Yc")
    return ops


def test_noalloc_runs_the_row_reduction_epilogue(monkeypatch):
    """The matmul -> reduction epilogue in its workspace form (row blocks
    combined across workgroups through counters in the flag words) from both
    entry points, on two calls in a row, the second smaller: the same matmul
    output and row maxima."""
    from metellus_amd.orchestrator import fusion

    hip_backend.init()
    monkeypatch.setattr(fusion, "MATMUL_REDUCTION_EPILOGUES", True)
    for shape, seed in (((512, 64, 1024), 41), ((300, 70, 520), 42)):
        print(f"noalloc: row max epilogue {shape}", flush=True)
        ops = _row_max_program(*shape, seed)
        (g,) = compile_program(ops)
        ws = g.kernel.workspace_bytes
        assert 0 < ws <= SCRATCH_MAX and "mt_rr_finish<" in g.kernel.source.split('extern "C"')[-1]
        inputs = {k: Buffer.from_numpy(a) for k, a in ops.uploads.items()}
        got = []
        for noalloc in (False, True):
            outs = {k: Buffer(ops.tensors[k].nbytes) for k in g.bindings if k not in inputs}
            for b in outs.values():
                b.fill(0xFF)  # NaN pattern: every element must be written
            bufs = [inputs[k] if k in inputs else outs[k] for k in g.bindings]
            args = (g.kernel.handle, bufs, g.dims, g.kernel.dims_slot_index, g.grid, g.threads)
            if noalloc:
                _noalloc_call(args, ws)
            else:
                hip_backend.launch(*args, workspace=ws)
                hip_backend.check_workspace()
            got.append({k: b.numpy(ops.tensors[k].shape, np.float32) for k, b in outs.items()})
            for b in outs.values():
                b.release()
        for b in inputs.values():
            b.release()
        a, b = got
        assert not np.isnan(a["r"]).any() and not np.isnan(a["Yc"]).any()
        for k in a:
            np.testing.assert_array_equal(a[k], b[k])
        np.testing.assert_array_equal(a["r"], a["Yc"].max(axis=1))


def fresh_process_check() -> None:
    """Run in a process of its own: an allocation-free call before any
    mt_launch has created the shim's workspace allocates nothing and creates
    no workspace; its output then matches mt_launch's bit for bit."""
    config.PERSISTENT, config.PERSISTENT_CAPACITY, config.STREAM_K = True, 5, True
    hip_backend.init()
    assert hip_backend.alloc_stats()["workspace_bytes"] == 0
    ops = gpu_cases.plain_matmul(1024, 256, 1024, seed=34)
    (g,) = compile_program(ops)
    ws = g.kernel.workspace_bytes
    assert ws > 0
    inputs = {k: Buffer.from_numpy(a) for k, a in ops.uploads.items()}
    outs = []
    for noalloc in (True, False):
        out = Buffer(1024 * 1024 * 4)
        out.fill(0xFF)
        bufs = [inputs[k] if k in inputs else out for k in g.bindings]
        args = (g.kernel.handle, bufs, g.dims, g.kernel.dims_slot_index, g.grid, g.threads)
        if noalloc:
            _noalloc_call(args, ws)
            assert hip_backend.alloc_stats()["workspace_bytes"] == 0
        else:
            hip_backend.launch(*args, workspace=ws)
            hip_backend.check_workspace()
            assert hip_backend.alloc_stats()["workspace_bytes"] >= ws
        outs.append(out.numpy((1024, 1024), np.float32))
    assert not np.isnan(outs[0]).any()
    np.testing.assert_array_equal(outs[0], outs[1])
    print("fresh-process no-alloc check: ok", flush=True)


def test_noalloc_first_call_in_a_fresh_process():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc: fresh process, no workspace yet", flush=True)
    r = subprocess.run(
        [sys.executable, "-c", "from tests.test_zz_no_alloc import fresh_process_check; fresh_process_check()"],
        cwd=root, capture_output=True, text=True, timeout=110,
    )
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "fresh-process no-alloc check: ok" in r.stdout
