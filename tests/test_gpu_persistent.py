"""Persistent tile loop on the GPU: forcing a small resident capacity makes
every matmul kernel loop over several tiles per workgroup (with the
cross-tile prefetch).  The per-tile arithmetic is unchanged, so the results
must be bit-identical to the one-tile-per-workgroup launch, and within the
matmul bar of the oracle.  Stream-K (which splits the last partial round by
k-chunks and so sums those tiles in another order) is switched off here and
tested in test_gpu_stream_k.py."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import run, run_batch
from metellus_amd.compute.matmul import config
from metellus_amd.orchestrator import Operations
from oracle.ir_eval import evaluate, matmul_tolerance
from tests import gpu_cases

pytestmark = pytest.mark.gpu


def _both(make, capacity, monkeypatch, runner=run):
    monkeypatch.setattr(config, "PERSISTENT", False)
    classic = runner(make())
    monkeypatch.setattr(config, "PERSISTENT", True)
    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", capacity)
    monkeypatch.setattr(config, "STREAM_K", False)
    persistent = runner(make())
    return classic, persistent


@pytest.mark.parametrize("mkn,capacity", [((192, 96, 320), 2), ((300, 72, 520), 3), ((1024, 256, 1024), 5)])
def test_plain_matmul_bit_identical(mkn, capacity, monkeypatch):
    M, K, N = mkn
    classic, persistent = _both(lambda: gpu_cases.plain_matmul(M, K, N, seed=7), capacity, monkeypatch)
    assert persistent.groups[0].grid == (capacity, 1, 1)
    assert classic.groups[0].grid[0] * classic.groups[0].grid[1] > capacity
    np.testing.assert_array_equal(persistent.env["C"], classic.env["C"])
    ops = gpu_cases.plain_matmul(M, K, N, seed=7)
    a, b = ops.uploads["A"], ops.uploads["B"]
    err = np.abs(persistent.env["C"].astype(np.float64) - evaluate(ops)["C"])
    assert np.all(err <= matmul_tolerance(a, b) + 1e-30)


def _prologue_epilogue_program():
    """Deferred broadcast prologue on A, register epilogue with a row
    operand, ragged M/N."""
    rng = np.random.default_rng(21)
    M, K, N = 150, 72, 170
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal(M).astype(np.float32), "mu")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    ops.from_numpy(rng.standard_normal(N).astype(np.float32), "bias")
    ops.reshape("mu", (M, 1), out="mu_c")
    ops.reshape("bias", (1, N), out="bias_r")
    ops.elementwise("subtract", out="a1", operands=("A", "mu_c"), y_broadcast="col")
    ops.matmul(a="a1", b="B", out="C")
    ops.elementwise("add", out="Cb", operands=("C", "bias_r"), y_broadcast="row")
    ops.elementwise("max", out="y", operands=("Cb", 0.0))
    return ops


def test_prologue_and_epilogue_bit_identical(monkeypatch):
    classic, persistent = _both(_prologue_epilogue_program, 2, monkeypatch)
    assert len(persistent.groups) == 1 and persistent.groups[0].grid == (2, 1, 1)
    np.testing.assert_array_equal(persistent.env["y"], classic.env["y"])
    ref = evaluate(_prologue_epilogue_program())
    tol = matmul_tolerance(ref["a1"], _prologue_epilogue_program().uploads["B"]) + 1e-30
    assert np.all(np.abs(persistent.env["y"] - ref["y"]) <= tol)


def test_batched_attention_bit_identical(monkeypatch):
    def make():
        return [gpu_cases.attention_head(256, 64, head=h, heads=3) for h in range(3)]

    classic, persistent = _both(make, 4, monkeypatch, runner=run_batch)
    for c, p in zip(classic, persistent):
        assert p.groups[0].grid == (1, 1, 1)  # capacity 4 over 3 programs: one looping workgroup each
        np.testing.assert_array_equal(p.env["O"], c.env["O"])
        np.testing.assert_array_equal(p.env["m1"], c.env["m1"])


def test_diamond_bit_identical(monkeypatch):
    """The shared-A multi-anchor kernel in a persistent tile loop."""
    classic, persistent = _both(lambda: gpu_cases.mlp_block(512, 256, 704, seed=6, diamond=True), 3, monkeypatch)
    assert len(persistent.groups) == 1 and persistent.groups[0].grid == (3, 1, 1)
    assert classic.groups[0].grid[0] * classic.groups[0].grid[1] > 3
    np.testing.assert_array_equal(persistent.env["z"], classic.env["z"])
