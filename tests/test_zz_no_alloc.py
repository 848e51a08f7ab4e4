"""The allocation-free launch (``mt_launch_noalloc``) through the C ABI,
against ``mt_launch`` with the shim's allocated workspace: stream-K matmul
kernels (the kernels that use a scratch buffer) give bit-identical outputs
from both entry points, on consecutive calls that shrink -- C4's X @ W1 at
its full size with the real resident capacity (the whole 64 MiB of partial
tiles), then smaller forced-capacity matmuls and a diamond with two
accumulator sets, whose calls reuse the same scratch.  The scratch error
word stays 0, and a request beyond the scratch's size is refused before
anything is launched."""

from __future__ import annotations

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
            assert hip_backend.launch_noalloc(*args, scratch=ws) == 0
        else:
            hip_backend.launch(*args, workspace=ws)
            hip_backend.check_workspace()
        outs.append(out.numpy(shape, np.float32))
        out.release()
    for b in inputs.values():
        b.release()
    return outs


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
