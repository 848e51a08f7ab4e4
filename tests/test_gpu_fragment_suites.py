"""The reference's fragment-level benches, restated on the MI355X: init
(tests/bench_init.py:46-113), one-row-per-workgroup reductions with 256
lanes (tests/bench_reduction.py:129-134), single-op elementwise over LDS
tiles with 32 x 8 workgroups (tests/bench_elementwise.py:277-329) and GEMMs
composed from matmul fragments over the reference's shape list
(tests/bench_matmul.py:195-208).  The reference compares against MLX with
rtol/atol 1e-5 (elementwise), 1e-4/1e-3 (sum, product), 1e-3/1e-2 (matmul);
the bars here are at least as strict:

* fill, copy, arange (mul then add, each rounded to fp32), IEEE-exact
  elementwise ops, max/min reductions: exact;
* sum/product reductions: bit-identical to the oracle's replay of the
  kernel's combine order;
* other elementwise ops: rtol = atol = 1e-5;
* matmul: |err| <= 1e-4 * sqrt(K) * (|A| @ |B|) elementwise.
"""

from __future__ import annotations

import numpy as np
import pytest

from compute.elementwise import elementwise_arity
from metellus_amd.compute.elementwise.elementwise import IEEE_EXACT_OPS
from oracle.ir_eval import UNARY, BINARY, matmul_tolerance, ordered_row_reduce
from runtime import Allocate, Dispatch, Download, Fill, FromNumpy, Runtime
from tests import fragment_kernels as fk

pytestmark = pytest.mark.gpu


def _run_1d(kernel, n, inputs=()):
    steps = [*(FromNumpy(name, arr) for name, arr in inputs), Allocate("Out", n * 4), kernel,
             Fill("Out", 0xFF),
             Dispatch(kernel, bindings=("Out", *(name for name, _ in inputs)), dims=(n,),
                      grid=fk.init_grid(n), threads=(fk.TG_X, 1, 1)),
             Download("Out", shape=(n,), dtype=np.float32, into="out")]
    return Runtime(tuple(steps)).run()["out"]


@pytest.mark.parametrize("n", [1, 256, 1000, 1024, 4097])
def test_fill(n):
    np.testing.assert_array_equal(_run_1d(fk.fill_kernel(3.5), n), np.full(n, 3.5, dtype=np.float32))


@pytest.mark.parametrize("n,start,step", [(1024, 0.0, 1.0), (1000, 5.0, 0.25), (4097, -2.0, 0.5)])
def test_arange(n, start, step):
    out = _run_1d(fk.arange_kernel(start, step), n)
    expected = np.float32(start) + np.float32(step) * np.arange(n, dtype=np.float32)
    np.testing.assert_array_equal(out, expected)


@pytest.mark.parametrize("n", [1, 1024, 1000, 4097])
def test_copy(n):
    src = np.linspace(-1.0, 1.0, n, dtype=np.float32)
    np.testing.assert_array_equal(_run_1d(fk.copy_kernel(), n, (("In", src),)), src)


@pytest.mark.parametrize("op", ["sum", "max", "min", "product"])
def test_single_workgroup_reductions(op):
    rng = np.random.default_rng(23)
    x = rng.uniform(0.75, 1.25, size=(17, 257)).astype(np.float32)
    m, n = x.shape
    kernel = fk.reduction_kernel(op)
    env = Runtime((
        FromNumpy("X", x), Allocate("Out", m * 4), kernel, Fill("Out", 0),
        Dispatch(kernel, bindings=("X", "Out"), dims=(m, n), grid=(m, 1, 1), threads=(fk.TG_X, 1, 1)),
        Download("Out", shape=(m,), dtype=np.float32, into="out"),
    )).run()
    out = env["out"]
    if op in ("max", "min"):
        np.testing.assert_array_equal(out, getattr(np, op)(x, axis=-1))
    else:
        # 256 lanes = 4 waves per row, symbolic N: per-element loop
        np.testing.assert_array_equal(out, ordered_row_reduce(x, op, waves_per_row=4, vectorized=False))
        ref = np.sum(x.astype(np.float64), axis=-1) if op == "sum" else np.prod(x.astype(np.float64), axis=-1)
        np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-3)


def _run_elementwise(op, x, y=None, cond=None, y_broadcast="none", cond_broadcast="none"):
    M, N = x.shape
    kernel, bindings, dims, grid, threads = fk.elementwise_kernel(
        op, M, N, y.shape if y is not None else None, cond.shape if cond is not None else None,
        y_broadcast, cond_broadcast)
    steps = [FromNumpy("X", x)]
    if y is not None:
        steps.append(FromNumpy("Y", y))
    if cond is not None:
        steps.append(FromNumpy("Cond", cond))
    steps += [Allocate("Out", M * N * 4), kernel, Fill("Out", 0),
              Dispatch(kernel, bindings=bindings, dims=dims, grid=grid, threads=threads),
              Download("Out", shape=(M, N), dtype=np.float32, into="out")]
    return Runtime(tuple(steps)).run()["out"]


def _check(op, out, ref):
    ref = np.asarray(ref).astype(np.float32)
    if op in IEEE_EXACT_OPS:
        np.testing.assert_array_equal(out, ref)
    else:
        np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


X = np.linspace(0.25, 3.75, 130, dtype=np.float32).reshape(10, 13)
Y = np.linspace(1.25, 2.25, 130, dtype=np.float32).reshape(10, 13)


@pytest.mark.parametrize("op", fk.UNARY_OPS)
def test_unary_ops(op):
    _check(op, _run_elementwise(op, X), UNARY[op](X))


@pytest.mark.parametrize("op", fk.BINARY_OPS)
def test_binary_ops(op):
    _check(op, _run_elementwise(op, X, Y), BINARY[op](X, Y))


def test_broadcast_ops():
    scalar = np.array([[2.0]], dtype=np.float32)
    row = np.linspace(1.0, 2.0, 13, dtype=np.float32).reshape(1, 13)
    col = np.linspace(1.0, 2.0, 10, dtype=np.float32).reshape(10, 1)
    np.testing.assert_array_equal(_run_elementwise("add", X, scalar, y_broadcast="scalar"), X + scalar)
    np.testing.assert_array_equal(_run_elementwise("add", X, row, y_broadcast="row"), X + row)
    np.testing.assert_array_equal(_run_elementwise("mul", X, col, y_broadcast="col"), X * col)


def test_where():
    y = np.flip(X, axis=1).copy()
    cond = (X > 2.0).astype(np.float32)
    np.testing.assert_array_equal(_run_elementwise("where", X, y, cond), np.where(cond != 0, X, y))


@pytest.mark.parametrize("shape", fk.GEMM_SHAPES)
def test_gemm_from_fragments(shape):
    m, k, n = shape
    rng = np.random.default_rng(m * 1_000_003 + k * 9_176 + n)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((k, n), dtype=np.float32)
    kernel, tile, aligned, grid = fk.gemm_kernel(m, k, n)
    env = Runtime((
        FromNumpy("A", a), FromNumpy("B", b), Allocate("C", m * n * 4), kernel, Fill("C", 0xFF),
        Dispatch(kernel, bindings=("A", "B", "C"), dims=(m, k, n), grid=grid, threads=(tile.tg_x, tile.tg_y, 1)),
        Download("C", shape=(m, n), dtype=np.float32, into="C_out"),
    )).run()
    err = np.abs(env["C_out"].astype(np.float64) - a.astype(np.float64) @ b.astype(np.float64))
    assert np.all(err <= matmul_tolerance(a, b) + 1e-30), f"max err {err.max():.3e} ({'aligned' if aligned else 'C tile'})"
