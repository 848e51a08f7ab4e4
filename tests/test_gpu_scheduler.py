"""End-to-end runs through ``schedule`` + ``Runtime`` on the GPU
(the reference's tests/test_scheduler.py, re-stated): outputs land in env,
fused intermediates never do, multi-consumer intermediates are materialised
and freed after their last reader, transposed views download exactly."""

import numpy as np
import pytest

from metellus_amd.api import compile_program, run
from metellus_amd.orchestrator import Operations
from metellus_amd.orchestrator.scheduler import schedule
from oracle.ir_eval import evaluate, matmul_tolerance
from tests import gpu_cases

pytestmark = pytest.mark.gpu


def _mm_ok(out, a, b, ref):
    assert np.all(np.abs(out.astype(np.float64) - ref) <= matmul_tolerance(a, b) + 1e-12)


def _ab(seed, M=32, K=16, N=24):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((M, K)).astype(np.float32), rng.standard_normal((K, N)).astype(np.float32)


def test_single_matmul():
    a, b = _ab(0)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(b, "B")
    ops.matmul(a="A", b="B", out="C")
    env = schedule(ops, compile_program(ops)).run()
    _mm_ok(env["C"], a, b, a.astype(np.float64) @ b)


def test_relu_fused_and_intermediate_absent():
    a, b = _ab(1)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(b, "B")
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("max", out="D", operands=("C", 0.0))
    groups = compile_program(ops)
    assert len(groups) == 1
    env = schedule(ops, groups).run()
    assert "C" not in env
    _mm_ok(env["D"], a, b, np.maximum(a.astype(np.float64) @ b, 0))


def test_two_consumers_materialise_intermediate():
    a, b = _ab(1)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(b, "B")
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("max", out="D", operands=("C", 0.0))
    ops.elementwise("absolute", out="E", operands=("C",))
    groups = compile_program(ops)
    assert len(groups) == 3
    env = schedule(ops, groups).run()
    c = a.astype(np.float64) @ b
    _mm_ok(env["C"], a, b, c)
    np.testing.assert_array_equal(env["D"], np.maximum(env["C"], 0))
    np.testing.assert_array_equal(env["E"], np.abs(env["C"]))


def test_two_independent_matmuls():
    rng = np.random.default_rng(2)
    mats = [rng.standard_normal((16, 16)).astype(np.float32) for _ in range(4)]
    ops = Operations()
    for n, m in zip("ABCD", mats):
        ops.from_numpy(m, n)
    ops.matmul(a="A", b="B", out="AB")
    ops.matmul(a="C", b="D", out="CD")
    groups = compile_program(ops)
    assert len(groups) == 2
    env = schedule(ops, groups).run()
    _mm_ok(env["AB"], mats[0], mats[1], mats[0].astype(np.float64) @ mats[1])
    _mm_ok(env["CD"], mats[2], mats[3], mats[2].astype(np.float64) @ mats[3])


def test_exp_relu_register_epilogue():
    a, b = _ab(3, 64, 32, 48)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(b, "B")
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("exp", out="E", operands=("C",))
    ops.elementwise("max", out="D", operands=("E", 0.0))
    groups = compile_program(ops)
    assert len(groups) == 1
    env = schedule(ops, groups).run()
    assert "C" not in env and "E" not in env
    np.testing.assert_allclose(env["D"], np.maximum(np.exp(a.astype(np.float64) @ b), 0), rtol=1e-3, atol=1e-3)


def test_transposed_view_download_is_exact():
    rng = np.random.default_rng(4)
    a = rng.standard_normal((8, 6)).astype(np.float32)
    b = rng.standard_normal((8, 5)).astype(np.float32)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(b, "B")
    ops.transpose("A", out="At")
    ops.matmul(a="At", b="B", out="C")
    env = schedule(ops, compile_program(ops)).run()
    np.testing.assert_array_equal(env["At"], a.T)
    _mm_ok(env["C"], a.T, b, a.T.astype(np.float64) @ b)


def test_profile_records_kernel_times():
    a, b = _ab(5)
    ops = Operations()
    ops.from_numpy(a, "A")
    ops.from_numpy(b, "B")
    ops.matmul(a="A", b="B", out="C")
    env = schedule(ops, compile_program(ops), profile=True).run()
    assert env["t_0"] > 0.0


def test_kernel_cache_hits_on_repeat():
    from metellus_amd.runtime import hip_backend

    a, b = _ab(6)
    for _ in range(2):
        ops = Operations()
        ops.from_numpy(a, "A")
        ops.from_numpy(b, "B")
        ops.matmul(a="A", b="B", out="C")
        before = hip_backend.cache_stats()
        schedule(ops, compile_program(ops)).run()
    after = hip_backend.cache_stats()
    assert after[0] == before[0]  # second run compiled nothing new


def test_large_downloads_land_in_pinned_pool_memory():
    import ctypes

    from metellus_amd.runtime.host import PINNED_MIN_BYTES

    ops = gpu_cases.sigmoid_chain(1024, 1024)  # 4 MiB output
    first = run(ops).env["out"]
    base = first.base
    while base is not None and not isinstance(base, ctypes.Array):
        base = getattr(base, "base", None)
    assert isinstance(base, ctypes.Array) and first.nbytes >= PINNED_MIN_BYTES
    ref = evaluate(ops)["out"]
    np.testing.assert_allclose(first, ref, rtol=1e-5, atol=1e-5)
    kept = first.copy()
    # blocks go back to the pool and are reused; earlier results stay intact
    for _ in range(3):
        again = run(ops).env["out"]
        np.testing.assert_array_equal(again, kept)
    np.testing.assert_array_equal(first, kept)
    del first, again
    np.testing.assert_array_equal(run(ops).env["out"], kept)


def test_outputs_selects_downloads():
    ops = gpu_cases.softmax(64, 256)
    full = run(ops).env
    only = run(ops, outputs=["p"]).env
    assert set(only) == {"p"}
    np.testing.assert_array_equal(only["p"], full["p"])
