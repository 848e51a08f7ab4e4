"""Partitions of the five BASELINE.json configs at their full sizes.

The strategy lists, op groupings, bindings and dims follow the hand trace of
the reference's rules (no reference run was possible: it needs Python 3.12
and Metal).  Launch shapes and LDS budgets are this backend's gfx950 tile
policy; every kernel must fit the 160 KiB LDS cap."""

from metellus_amd.api import compile_program
from metellus_amd.orchestrator.aliasing import TGMEM_CAP_BYTES, compute_group_budget
from metellus_amd.orchestrator.kernel_group import FusionStrategy as S
from metellus_amd.orchestrator import Operations


def _inputs(ops, **shapes):
    for name, shape in shapes.items():
        ops.input(name, shape=shape)


def c1():
    ops = Operations()
    _inputs(ops, A=(256, 256), B=(256, 256), bias=(256,))
    ops.reshape("bias", (1, 256), out="bias_row")
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("add", out="Cb", operands=("C", "bias_row"), y_broadcast="row")
    ops.elementwise("max", out="y", operands=("Cb", 0.0))
    return ops


def c2():
    ops = Operations()
    _inputs(ops, a=(4096, 4096), b=(4096, 4096), c=(4096, 4096), d=(4096, 4096))
    ops.elementwise("mul", out="t1", operands=("a", "b"))
    ops.elementwise("add", out="t2", operands=("t1", "c"))
    ops.elementwise("negate", out="n", operands=("t2",))
    ops.elementwise("exp", out="e", operands=("n",))
    ops.elementwise("add", out="p", operands=("e", 1.0))
    ops.elementwise("recip", out="s", operands=("p",))
    ops.elementwise("mul", out="out", operands=("s", "d"))
    return ops


def c3():
    ops = Operations()
    _inputs(ops, x=(8192, 8192))
    ops.reduction("max", out="m1", x="x")
    ops.reshape("m1", (8192, 1), out="m")
    ops.elementwise("subtract", out="sh", operands=("x", "m"), y_broadcast="col")
    ops.elementwise("exp", out="e", operands=("sh",))
    ops.reduction("sum", out="s1", x="e")
    ops.reshape("s1", (8192, 1), out="sv")
    ops.elementwise("div", out="p", operands=("e", "sv"), y_broadcast="col")
    return ops


def c4(diamond=False):
    ops = Operations()
    _inputs(ops, X=(4096, 4096), W1=(4096, 11008), W2=(4096, 11008))
    ops.matmul(a="X", b="W1", out="h1")
    ops.matmul(a="X", b="W2", out="h2")
    if diamond:
        ops.elementwise("mul", out="z", operands=("h1", "h2"))
        return ops
    ops.input("W3", shape=(11008, 4096))
    ops.elementwise("negate", out="n", operands=("h1",))
    ops.elementwise("exp", out="e", operands=("n",))
    ops.elementwise("add", out="p", operands=("e", 1.0))
    ops.elementwise("recip", out="s", operands=("p",))
    ops.elementwise("mul", out="g", operands=("h1", "s"))
    ops.elementwise("mul", out="z", operands=("g", "h2"))
    ops.matmul(a="z", b="W3", out="out")
    return ops


def c5_head():
    ops = Operations()
    _inputs(ops, Q=(2048, 128), K=(2048, 128), V=(2048, 128))
    ops.transpose("K", out="Kt")
    ops.matmul(a="Q", b="Kt", out="S")
    ops.elementwise("mul", out="Ss", operands=("S", 0.08838834764831845))
    ops.reduction("max", out="m1", x="Ss")
    ops.reshape("m1", (2048, 1), out="m")
    ops.elementwise("subtract", out="sh", operands=("Ss", "m"), y_broadcast="col")
    ops.elementwise("exp", out="e", operands=("sh",))
    ops.reduction("sum", out="s1", x="e")
    ops.reshape("s1", (2048, 1), out="sv")
    ops.elementwise("div", out="P", operands=("e", "sv"), y_broadcast="col")
    ops.matmul(a="P", b="V", out="O")
    return ops


def _summary(ops):
    gs = compile_program(ops)
    for g in gs:
        assert compute_group_budget(g).size_bytes <= TGMEM_CAP_BYTES
    return gs


def test_c1_one_kernel():
    (g,) = _summary(c1())
    assert g.strategy is S.MATMUL_EPILOGUE_TG
    assert g.bindings == ("A", "B", "y", "bias") and g.dims == (256, 256, 256)
    assert [op.out.name for op in g.ops] == ["C", "Cb", "y"]


def test_c2_one_chain():
    (g,) = _summary(c2())
    assert g.strategy is S.ELEMENTWISE_CHAIN and len(g.ops) == 7
    assert g.bindings == ("a", "out", "b", "c", "d") and g.dims == (4096, 4096)
    assert compute_group_budget(g).size_bytes == 0  # register-resident


def test_c3_four_kernels():
    gs = _summary(c3())
    assert [g.strategy for g in gs] == [
        S.STANDALONE_REDUCTION, S.ELEMENTWISE_CHAIN, S.STANDALONE_REDUCTION, S.STANDALONE_ELEMENTWISE
    ]
    assert [g.bindings for g in gs] == [("x", "m1"), ("x", "e", "m1"), ("e", "s1"), ("e", "p", "s1")]
    assert all(g.dims == (8192, 8192) for g in gs)


def test_c4_literal_four_kernels():
    gs = _summary(c4())
    assert [g.strategy for g in gs] == [
        S.STANDALONE_MATMUL, S.STANDALONE_MATMUL, S.ELEMENTWISE_CHAIN, S.ELEMENTWISE_PROLOGUE_MATMUL
    ]
    assert gs[0].bindings == ("X", "W1", "h1") and gs[1].bindings == ("X", "W2", "h2")
    assert gs[2].bindings == ("h1", "s")
    assert gs[3].bindings == ("h1", "W3", "out", "s", "h2")
    assert gs[3].dims == (4096, 11008, 4096)
    # 256x256 tiles: 43 x 16 = 688 tiles > 256 resident workgroups, so the
    # GEMM runs as 256 persistent workgroups of 16 waves; X @ W3 (its
    # prologue gathers the full-size s and h2) has exactly 256 tiles, 8 waves
    assert gs[0].grid == (256, 1, 1) and gs[0].threads == (1024, 1, 1)
    assert gs[3].grid == (16, 16, 1) and gs[3].threads == (512, 1, 1)


def test_c4_diamond_fuses_under_160k():
    (g,) = _summary(c4(diamond=True))
    assert g.strategy is S.DIAMOND_SHARED
    assert g.bindings == ("X", "W1", "W2", "z") and g.dims == (4096, 4096, 11008)
    # 256x128 tiles, dense: A 2x256x32 + two B chunks 2x32x128 floats
    assert compute_group_budget(g).size_bytes == 131_072


def test_c5_five_kernels_per_head():
    gs = _summary(c5_head())
    assert [g.strategy for g in gs] == [
        S.MATMUL_EPILOGUE_REGISTER,
        S.STANDALONE_REDUCTION,
        S.ELEMENTWISE_CHAIN,
        S.STANDALONE_REDUCTION,
        S.ELEMENTWISE_PROLOGUE_MATMUL,
    ]
    assert gs[0].bindings == ("Q", "K", "Ss")  # K^T is a view of K: no transpose kernel
    assert gs[4].bindings == ("e", "V", "O", "s1")
