"""GPU parity: every strategy family through ``api.run`` on the MI355X,
checked against the CPU oracle (``oracle/ir_eval.py``).

Bars (stated per check):
* IEEE-exact elementwise ops, max/min reductions, copies: exact equality;
* sum/product reductions: bit-identical to the oracle's replay of the
  kernel's combine order (``ordered_row_reduce``), and within 1e-5 of the
  float64 sum;
* chains with transcendentals (exp, log, tanh, ...): rtol = atol = 1e-5;
* matmul: |err| <= 1e-4 * sqrt(K) * (|A| @ |B|) elementwise.
"""

from __future__ import annotations

import numpy as np
import pytest

from metellus_amd.api import run
from metellus_amd.orchestrator import Operations
from metellus_amd.orchestrator.assembly.reduction import reduction_order
from metellus_amd.orchestrator.kernel_group import FusionStrategy
from oracle.ir_eval import evaluate, matmul_tolerance, ordered_row_reduce
from tests import gpu_cases

pytestmark = pytest.mark.gpu


def _check_matmul(out, a, b, ref):
    err = np.abs(out.astype(np.float64) - ref)
    tol = matmul_tolerance(a, b) + 1e-30
    bad = err > tol
    assert not bad.any(), f"{bad.sum()} elements over tolerance; max err {err.max():.3e}"


# ---------------------------------------------------------------------------
# elementwise
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("shape", [(96, 160), (37, 41), (1024, 1024), (1, 7)])
def test_sigmoid_chain(shape):
    ops = gpu_cases.sigmoid_chain(*shape)
    res = run(ops)
    assert [g.strategy for g in res.groups] == [FusionStrategy.ELEMENTWISE_CHAIN]
    ref = evaluate(ops)["out"]
    np.testing.assert_allclose(res.env["out"], ref, rtol=1e-5, atol=1e-5)


def test_exact_chain_is_bit_exact():
    """IEEE-exact ops only: (a*b + c) / d - max(a, 0) must match exactly."""
    rng = np.random.default_rng(11)
    ops = Operations()
    for n in "abcd":
        ops.from_numpy(rng.standard_normal((64, 200)).astype(np.float32), n)
    ops.elementwise("mul", out="t1", operands=("a", "b"))
    ops.elementwise("add", out="t2", operands=("t1", "c"))
    ops.elementwise("div", out="t3", operands=("t2", "d"))
    ops.elementwise("sqrt", out="t4", operands=("t3",))
    ops.elementwise("subtract", out="out", operands=("t4", "a"))
    res = run(ops)
    ref = evaluate(ops)["out"]
    np.testing.assert_array_equal(res.env["out"], ref)


@pytest.mark.parametrize("mode", ["row", "col", "scalar"])
def test_broadcast_operands(mode):
    rng = np.random.default_rng(5)
    M, N = 48, 72
    shapes = {"row": (1, N), "col": (M, 1), "scalar": (1, 1)}
    ops = Operations()
    ops.from_numpy(rng.standard_normal((M, N)).astype(np.float32), "X")
    ops.from_numpy(rng.standard_normal(shapes[mode]).astype(np.float32), "Y")
    ops.elementwise("mul", out="Z", operands=("X", "Y"), y_broadcast=mode)
    ops.elementwise("add", out="W", operands=("Z", 0.5))
    res = run(ops)
    np.testing.assert_array_equal(res.env["W"], evaluate(ops)["W"])


def test_strided_secondary_view():
    """Y is a transposed view: read through strides (1, 4)."""
    rng = np.random.default_rng(6)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((4, 8)).astype(np.float32), "X")
    ops.from_numpy(rng.standard_normal((8, 4)).astype(np.float32), "Ybase")
    ops.transpose("Ybase", out="Y")
    ops.elementwise("add", out="Z", operands=("X", "Y"))
    res = run(ops)
    np.testing.assert_array_equal(res.env["Z"], evaluate(ops)["Z"])


def test_where_and_comparisons():
    rng = np.random.default_rng(7)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((40, 64)).astype(np.float32), "X")
    ops.from_numpy(rng.standard_normal((40, 64)).astype(np.float32), "Y")
    ops.elementwise("gt", out="mask", operands=("X", 0.0))
    ops.elementwise("where", out="W", operands=("X", "Y", "mask"))
    res = run(ops)
    np.testing.assert_array_equal(res.env["W"], evaluate(ops)["W"])


# ---------------------------------------------------------------------------
# reductions
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("shape", [(64, 256), (8, 8192), (33, 100), (17, 257), (1024, 4096)])
@pytest.mark.parametrize("op", ["sum", "max", "min", "product"])
def test_reduction_exact_order(shape, op):
    rng = np.random.default_rng(23)
    lo, hi = (0.95, 1.05) if op == "product" else (-1.0, 1.0)
    x = rng.uniform(lo, hi, size=shape).astype(np.float32)
    ops = Operations()
    ops.from_numpy(x, "X")
    ops.reduction(op, out="R", x="X")
    res = run(ops)
    (g,) = res.groups
    order = reduction_order(g)
    replay = ordered_row_reduce(x, op, order["waves_per_row"], order["vectorized"])
    np.testing.assert_array_equal(res.env["R"], replay)
    ref = evaluate(ops)["R"]
    if op in ("sum", "product"):
        # float32 accumulation error bound against the float64 reference
        np.testing.assert_allclose(res.env["R"], ref, rtol=1e-4, atol=2e-7 * shape[1])
    else:
        np.testing.assert_array_equal(res.env["R"], ref)


def test_reduction_prologue_and_epilogue():
    rng = np.random.default_rng(9)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((32, 300)).astype(np.float32), "X")
    ops.elementwise("exp", out="EX", operands=("X",))
    ops.reduction("sum", out="S", x="EX")
    ops.elementwise("mul", out="Y", operands=("S", 0.5))
    res = run(ops)
    strategies = [g.strategy for g in res.groups]
    assert FusionStrategy.ELEMENTWISE_PROLOGUE_REDUCTION in strategies
    np.testing.assert_allclose(res.env["Y"], evaluate(ops)["Y"], rtol=1e-5)


@pytest.mark.parametrize("shape", [(64, 256), (8, 8192), (33, 100)])
def test_softmax(shape):
    ops = gpu_cases.softmax(*shape)
    res = run(ops)
    assert len(res.groups) == 4
    ref = evaluate(ops)
    np.testing.assert_array_equal(res.env["m1"], ref["m1"])  # max: exact
    np.testing.assert_allclose(res.env["e"], ref["e"], rtol=1e-5, atol=1e-6)
    # the sum kernel is checked against the replay of its order on the GPU's own e
    sum_group = res.groups[2]
    order = reduction_order(sum_group)
    replay = ordered_row_reduce(res.env["e"], "sum", order["waves_per_row"], order["vectorized"])
    np.testing.assert_array_equal(res.env["s1"], replay)
    np.testing.assert_allclose(res.env["p"], ref["p"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(res.env["p"].sum(axis=1), 1.0, rtol=1e-5)


# ---------------------------------------------------------------------------
# matmul family
# ---------------------------------------------------------------------------


@pytest.mark.parametrize(
    "mkn",
    [(256, 256, 256), (64, 32, 64), (100, 70, 130), (512, 512, 512), (1024, 1024, 1024), (4096, 256, 4096)],
)
def test_plain_matmul(mkn):
    M, K, N = mkn
    ops = gpu_cases.plain_matmul(M, K, N)
    res = run(ops)
    a, b = ops.uploads["A"], ops.uploads["B"]
    _check_matmul(res.env["C"], a, b, a.astype(np.float64) @ b.astype(np.float64))


def test_c1_matmul_bias_relu():
    ops = gpu_cases.matmul_bias_relu(256, 256, 256)
    res = run(ops)
    assert [g.strategy for g in res.groups] == [FusionStrategy.MATMUL_EPILOGUE_TG]
    a, b = ops.uploads["A"], ops.uploads["B"]
    _check_matmul(res.env["y"], a, b, evaluate(ops)["y"])


def test_register_epilogue_and_prologue():
    rng = np.random.default_rng(3)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((128, 96)).astype(np.float32), "A")
    ops.from_numpy(rng.standard_normal((96, 160)).astype(np.float32), "B")
    ops.elementwise("max", out="Ar", operands=("A", 0.0))
    ops.matmul(a="Ar", b="B", out="C")
    ops.elementwise("mul", out="D", operands=("C", 0.25))
    res = run(ops)
    assert len(res.groups) == 1
    a = np.maximum(ops.uploads["A"], 0)
    _check_matmul(res.env["D"], a, ops.uploads["B"] * 0.25, evaluate(ops)["D"])


@pytest.mark.parametrize("layout", ["rowmajor", "transposed", "transposed_odd"])
def test_broadcast_prologues_gathered(layout):
    """Prologues reading only broadcast operands load those operands with the
    tile (fetch_gather) and are applied when the tile is written to LDS
    (commit_apply), with 32-wide k-chunks.  A is loaded 128-bit along
    columns (row-major), 128-bit along rows (transposed view, column stride
    100) or element by element (transposed view, column stride 101); B
    (N = 90) by elements.  M, N are not tile multiples, so bounds apply."""
    rng = np.random.default_rng(12)
    M = 101 if layout == "transposed_odd" else 100
    K, N = 72, 90
    ops = Operations()
    if layout == "rowmajor":
        ops.from_numpy(rng.standard_normal((M, K)).astype(np.float32), "A")
    else:
        ops.from_numpy(rng.standard_normal((K, M)).astype(np.float32), "At")
        ops.transpose("At", out="A")
    ops.from_numpy(rng.standard_normal(M).astype(np.float32), "mu")
    ops.from_numpy(rng.uniform(0.5, 1.5, K).astype(np.float32), "g")
    ops.from_numpy(rng.standard_normal((K, N)).astype(np.float32), "B")
    ops.from_numpy(rng.uniform(0.5, 1.5, N).astype(np.float32), "h")
    ops.reshape("mu", (M, 1), out="mu_c")
    ops.reshape("g", (1, K), out="g_r")
    ops.reshape("h", (1, N), out="h_r")
    ops.elementwise("subtract", out="a1", operands=("A", "mu_c"), y_broadcast="col")
    ops.elementwise("mul", out="a2", operands=("a1", "g_r"), y_broadcast="row")
    ops.elementwise("mul", out="b1", operands=("B", "h_r"), y_broadcast="row")
    ops.matmul(a="a2", b="b1", out="C")
    res = run(ops)
    assert [g.strategy for g in res.groups] == [FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL]
    src = res.groups[0].kernel.source
    body = src.split('extern "C"')[1]
    # A and B loaders, each once before the k loop and once inside it
    assert body.count("fetch_gather<true>") == 4 and body.count("commit_apply<") == 4
    assert "fetch_raw<" not in src.split('extern "C"')[1]
    ref = evaluate(ops)
    _check_matmul(res.env["C"], ref["a2"], ref["b1"], ref["C"])


def test_transposed_operands():
    rng = np.random.default_rng(4)
    ops = Operations()
    ops.from_numpy(rng.standard_normal((96, 128)).astype(np.float32), "A")  # A^T is (128, 96)
    ops.from_numpy(rng.standard_normal((64, 96)).astype(np.float32), "Bb")  # Bb^T is (96, 64)
    ops.transpose("A", out="At")
    ops.transpose("Bb", out="B")
    ops.matmul(a="At", b="B", out="C")
    res = run(ops)
    a = ops.uploads["A"].T
    b = ops.uploads["Bb"].T
    _check_matmul(res.env["C"], a, b, evaluate(ops)["C"])


def test_diamond_and_multi_producer():
    ops = gpu_cases.mlp_block(256, 256, 512, diamond=True)
    res = run(ops)
    assert [g.strategy for g in res.groups] == [FusionStrategy.DIAMOND_SHARED]
    ref = evaluate(ops)
    x, w1, w2 = (ops.uploads[k].astype(np.float64) for k in ("X", "W1", "W2"))
    h1, h2 = x @ w1, x @ w2
    tol = 1e-4 * np.sqrt(256) * ((np.abs(x) @ np.abs(w1)) * np.abs(h2) + (np.abs(x) @ np.abs(w2)) * np.abs(h1)) + 1e-12
    assert np.all(np.abs(res.env["z"] - ref["z"]) <= tol)

    rng = np.random.default_rng(8)
    ops = Operations()
    for n, s in (("A", (128, 64)), ("B", (64, 96)), ("C", (128, 32)), ("D", (32, 96))):
        ops.from_numpy(rng.standard_normal(s).astype(np.float32), n)
    ops.matmul(a="A", b="B", out="c1")
    ops.matmul(a="C", b="D", out="c2")
    ops.elementwise("add", out="z", operands=("c1", "c2"))
    res = run(ops)
    assert [g.strategy for g in res.groups] == [FusionStrategy.MULTI_PRODUCER_CONVERGENT]
    ref = evaluate(ops)["z"]
    a, b, c, d = (ops.uploads[k] for k in "ABCD")
    tol = matmul_tolerance(a, b) + matmul_tolerance(c, d) + 1e-12
    assert np.all(np.abs(res.env["z"] - ref) <= tol)


def test_mlp_block_literal():
    ops = gpu_cases.mlp_block(128, 128, 384)
    res = run(ops)
    assert [g.strategy for g in res.groups] == [
        FusionStrategy.STANDALONE_MATMUL,
        FusionStrategy.STANDALONE_MATMUL,
        FusionStrategy.ELEMENTWISE_CHAIN,
        FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL,
    ]
    ref = evaluate(ops)
    np.testing.assert_allclose(res.env["out"], ref["out"], rtol=1e-3, atol=1e-4)


@pytest.mark.parametrize("S,Dh", [(256, 64), (100, 40)])
def test_attention_head(S, Dh):
    ops = gpu_cases.attention_head(S, Dh)
    res = run(ops)
    assert len(res.groups) == 5
    ref = evaluate(ops)
    # m1 is the max of a matmul output, so it inherits the matmul tolerance
    np.testing.assert_allclose(res.env["m1"], ref["m1"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(res.env["O"], ref["O"], rtol=1e-3, atol=1e-4)


# ---------------------------------------------------------------------------
# shape copy
# ---------------------------------------------------------------------------


@pytest.mark.parametrize(
    "shape,new",
    [
        ((8, 16), (128,)), ((8, 16), (32, 4)), ((10, 13), (130,)), ((32, 32), (1024,)),
        # LDS-tiled transpose copy: ragged 64x64 tiles in both axes, and a large one
        ((65, 130), (8450,)), ((300, 257), (514, 150)), ((4096, 1024), (4194304,)),
    ],
)
def test_shape_copy_exact(shape, new):
    rng = np.random.default_rng(0)
    x = rng.standard_normal(shape).astype(np.float32)
    ops = Operations()
    ops.from_numpy(x, "X")
    ops.transpose("X", out="Xt")
    ops.reshape("Xt", new, out="Y")
    res = run(ops)
    assert [g.strategy for g in res.groups] == [FusionStrategy.STANDALONE_SHAPE]
    np.testing.assert_array_equal(res.env["Y"], x.T.reshape(new))
