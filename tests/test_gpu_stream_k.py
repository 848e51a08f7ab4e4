"""Stream-K persistent matmuls on the GPU.  A small forced resident capacity
(or, for C4's X @ W1, the real one) leaves a partial last round, which runs
split by k-chunks with partial tiles handed over through the shim's
workspace.  Checked: every output within the matmul bar of the oracle,
launches reproducible bit for bit, the workspace flags left clean (back to
back launches of different programs stay correct, and the error word stays
0), and agreement with the plain persistent loop to the same bar."""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import run
from metellus_amd.compute.matmul import config
from metellus_amd.orchestrator import Operations
from metellus_amd.runtime import hip_backend
from oracle.ir_eval import evaluate, matmul_tolerance
from tests import gpu_cases

pytestmark = pytest.mark.gpu


def _stream_k(monkeypatch, capacity):
    monkeypatch.setattr(config, "PERSISTENT", True)
    monkeypatch.setattr(config, "PERSISTENT_CAPACITY", capacity)
    monkeypatch.setattr(config, "STREAM_K", True)


# (M, K, N), capacity: tiles not a whole number of rounds.  K = 128 (4
# k-chunks) on 7 workgroups gives ranges of 1-2 chunks, so a split tile has
# up to 4 contributors; 1000^3 is ragged in every dimension.
CASES = [
    ((192, 96, 320), 4),
    ((300, 72, 520), 4),
    ((1024, 256, 1024), 5),
    ((640, 128, 768), 7),
    ((1000, 1000, 1000), 6),
    ((2048, 512, 1536), 13),
]


@pytest.mark.parametrize("mkn,capacity", CASES)
def test_plain_matmul_within_bar_and_reproducible(mkn, capacity, monkeypatch):
    M, K, N = mkn
    print(f"stream-K plain matmul {mkn} capacity {capacity}", flush=True)
    _stream_k(monkeypatch, capacity)
    ops = gpu_cases.plain_matmul(M, K, N, seed=11)
    first = run(ops)
    g = first.groups[0]
    assert g.grid == (capacity, 1, 1) and g.kernel.workspace_bytes > 0
    second = run(gpu_cases.plain_matmul(M, K, N, seed=11))
    np.testing.assert_array_equal(first.env["C"], second.env["C"])
    a, b = ops.uploads["A"], ops.uploads["B"]
    err = np.abs(first.env["C"].astype(np.float64) - evaluate(ops)["C"])
    assert np.all(err <= matmul_tolerance(a, b) + 1e-30)
    hip_backend.check_workspace()


def test_agrees_with_plain_persistent_loop(monkeypatch):
    M, K, N = 1000, 1000, 1000
    _stream_k(monkeypatch, 6)
    sk = run(gpu_cases.plain_matmul(M, K, N, seed=12))
    monkeypatch.setattr(config, "STREAM_K", False)
    dp = run(gpu_cases.plain_matmul(M, K, N, seed=12))
    assert dp.groups[0].kernel.workspace_bytes == 0
    ops = gpu_cases.plain_matmul(M, K, N, seed=12)
    tol = matmul_tolerance(ops.uploads["A"], ops.uploads["B"]) + 1e-30
    assert np.all(np.abs(sk.env["C"].astype(np.float64) - dp.env["C"]) <= 2 * tol)
    # tiles finished inside one workgroup sum in the same order as the plain loop
    assert np.mean(sk.env["C"] == dp.env["C"]) > 0.5


def _prologue_epilogue_program(M=330, K=200, N=410, seed=21):
    """Broadcast prologue on A (deferred), full-size gather prologue on B,
    register epilogue with a row operand and a ReLU; ragged M/N."""
    rng = np.random.default_rng(seed)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal(M).astype(np.float32), "mu")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "G")
    ops.from_numpy(rng.standard_normal(N).astype(np.float32), "bias")
    ops.reshape("mu", (M, 1), out="mu_c")
    ops.reshape("bias", (1, N), out="bias_r")
    ops.elementwise("subtract", out="a1", operands=("A", "mu_c"), y_broadcast="col")
    ops.elementwise("mul", out="b1", operands=("B", "G"))
    ops.matmul(a="a1", b="b1", out="C")
    ops.elementwise("add", out="Cb", operands=("C", "bias_r"), y_broadcast="row")
    ops.elementwise("max", out="y", operands=("Cb", 0.0))
    return ops


def test_prologues_and_epilogue(monkeypatch):
    _stream_k(monkeypatch, 5)
    res = run(_prologue_epilogue_program())
    assert len(res.groups) == 1 and res.groups[0].kernel.workspace_bytes > 0
    ref = evaluate(_prologue_epilogue_program())
    tol = matmul_tolerance(ref["a1"], ref["b1"]) + 1e-30
    assert np.all(np.abs(res.env["y"] - ref["y"]) <= tol)


def test_back_to_back_programs_leave_flags_clean(monkeypatch):
    """Owners clear the flags they consume: launches of different schedules
    in a row each read only their own partial tiles."""
    _stream_k(monkeypatch, 7)
    for seed, (M, K, N) in enumerate([(640, 256, 768), (512, 1024, 900), (640, 256, 768), (900, 160, 300)]):
        ops = gpu_cases.plain_matmul(M, K, N, seed=30 + seed)
        res = run(ops)
        assert res.groups[0].kernel.workspace_bytes > 0
        err = np.abs(res.env["C"].astype(np.float64) - evaluate(ops)["C"])
        assert np.all(err <= matmul_tolerance(ops.uploads["A"], ops.uploads["B"]) + 1e-30), (M, K, N)
    hip_backend.check_workspace()


def test_c4_x_w1_at_full_size():
    """C4's X @ W1 (4096 x 4096 @ 4096 x 11008) with the real capacity: 688
    tiles, 512 data-parallel, 176 split over 256 workgroups.  Rows sampled
    from both parts are checked against float64 products."""
    ops = gpu_cases.mlp_block(4096, 4096, 11008, seed=3)
    res = run(ops, outputs=("h1",))
    g = [x for x in res.groups if x.kernel.function_name.startswith("matmul_h1")][0]
    assert g.grid == (256, 1, 1) and g.kernel.workspace_bytes > 0
    x, w1 = ops.uploads["X"].astype(np.float64), ops.uploads["W1"].astype(np.float64)
    rng = np.random.default_rng(0)
    rows = np.concatenate([rng.choice(2816, 24, replace=False), 2816 + rng.choice(1280, 40, replace=False)])
    ref = x[rows] @ w1
    tol = 1e-4 * np.sqrt(4096) * (np.abs(x[rows]) @ np.abs(w1)) + 1e-30
    assert np.all(np.abs(res.env["h1"][rows] - ref) <= tol)


@pytest.mark.parametrize("mdh,capacity", [((512, 256, 704), 5), ((700, 300, 900), 7)])
def test_diamond_two_accumulator_sets(mdh, capacity, monkeypatch):
    """(X @ W1) * (X @ W2) in one kernel: both accumulator sets of a split
    tile are handed over."""
    M, D, H = mdh
    _stream_k(monkeypatch, capacity)
    ops = gpu_cases.mlp_block(M, D, H, seed=5, diamond=True)
    first = run(ops)
    assert len(first.groups) == 1
    g = first.groups[0]
    assert g.grid == (capacity, 1, 1) and g.kernel.workspace_bytes > 0
    second = run(gpu_cases.mlp_block(M, D, H, seed=5, diamond=True))
    np.testing.assert_array_equal(first.env["z"], second.env["z"])
    ref = evaluate(ops)
    x, w1, w2 = (ops.uploads[k].astype(np.float64) for k in ("X", "W1", "W2"))
    h1, h2 = ref["h1"], ref["h2"]
    # |h1 h2 - z| <= |h2| tol(h1) + |h1| tol(h2) + tol(h1) tol(h2), tol = the matmul bar
    t1, t2 = matmul_tolerance(x, w1), matmul_tolerance(x, w2)
    bound = np.abs(h2) * t1 + np.abs(h1) * t2 + t1 * t2 + np.abs(h1 * h2) * 2.0 ** -23 + 1e-30
    assert np.all(np.abs(first.env["z"] - h1 * h2) <= bound)
