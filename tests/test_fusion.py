"""Fusion rules and assembly structure.

Restates the reference's tests/test_fusion.py: which ops land in which
vertex, the strategy label ``assemble`` gives each, bindings and dims.  The
reference's assertions on MSL text are retargeted to the HIP the gfx950
templates emit (stated per test)."""

from orchestrator import MatmulOp, Operations
from orchestrator.assembly import assemble
from orchestrator.fusion import fuse
from orchestrator.ir import ElementwiseOp, ReductionOp
from orchestrator.kernel_group import FusionStrategy


def _types(v):
    return [type(o).__name__ for o in v.ops]


def _around_anchor(v):
    idx = next((i for i, op in enumerate(v.ops) if isinstance(op, (MatmulOp, ReductionOp))), None)
    if idx is None:
        return None, None
    pre = [op for op in v.ops[:idx] if isinstance(op, ElementwiseOp)]
    post = [op for op in v.ops[idx + 1 :] if isinstance(op, ElementwiseOp)]
    return pre, post


def _bias_relu(M=32, K=64, N=128):
    ops = Operations()
    ops.input("A", shape=(M, K))
    ops.input("B", shape=(K, N))
    ops.input("bias", shape=(1, N))
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("add", out="D", operands=("C", "bias"), y_broadcast="row")
    ops.elementwise("max", out="Y", operands=("D", 0.0))
    return ops


def test_epilogue_tile_label_with_row_broadcast():
    (v,) = fuse(_bias_relu().build())
    assert _types(v) == ["MatmulOp", "ElementwiseOp", "ElementwiseOp"]
    pre, post = _around_anchor(v)
    assert pre == [] and len(post) == 2
    assert assemble(v).strategy is FusionStrategy.MATMUL_EPILOGUE_TG


def test_register_epilogue_for_lane_agnostic_chain():
    ops = Operations()
    ops.input("A", shape=(128, 64))
    ops.input("B", shape=(64, 128))
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("max", out="Y", operands=("C", 0.0))
    (v,) = fuse(ops.build())
    assert _types(v) == ["MatmulOp", "ElementwiseOp"]
    assert assemble(v).strategy is FusionStrategy.MATMUL_EPILOGUE_REGISTER


def test_prologues():
    ops = Operations()
    ops.input("A", shape=(128, 64))
    ops.input("B", shape=(64, 128))
    ops.elementwise("max", out="A_relu", operands=("A", 0.0))
    ops.matmul(a="A_relu", b="B", out="C")
    (v,) = fuse(ops.build())
    pre, post = _around_anchor(v)
    assert [op.op for op in pre] == ["max"] and post == []
    assert assemble(v).strategy is FusionStrategy.ELEMENTWISE_PROLOGUE_MATMUL

    ops = Operations()
    ops.input("X", shape=(32, 64))
    ops.elementwise("exp", out="EX", operands=("X",))
    ops.reduction("sum", out="S", x="EX")
    (v,) = fuse(ops.build())
    assert [op.op for op in _around_anchor(v)[0]] == ["exp"]
    assert assemble(v).strategy is FusionStrategy.ELEMENTWISE_PROLOGUE_REDUCTION


def test_reduction_epilogue_scalar_only():
    ops = Operations()
    ops.input("X", shape=(32, 64))
    ops.reduction("sum", out="S", x="X")
    ops.elementwise("mul", out="Y", operands=("S", 0.5))
    (v,) = fuse(ops.build())
    pre, post = _around_anchor(v)
    assert pre == [] and len(post) == 1
    assert assemble(v).strategy is FusionStrategy.REDUCTION_EPILOGUE


def test_elementwise_chain_and_standalone_matmul():
    ops = Operations()
    ops.input("X", shape=(32, 64))
    ops.elementwise("exp", out="E", operands=("X",))
    ops.elementwise("log", out="L", operands=("E",))
    (v,) = fuse(ops.build())
    assert _types(v) == ["ElementwiseOp", "ElementwiseOp"]
    assert assemble(v).strategy is FusionStrategy.ELEMENTWISE_CHAIN
    ops = Operations()
    ops.input("A", shape=(64, 64))
    ops.input("B", shape=(64, 64))
    ops.matmul(a="A", b="B", out="C")
    (v,) = fuse(ops.build())
    assert assemble(v).strategy is FusionStrategy.STANDALONE_MATMUL


def test_prologue_and_epilogue_around_one_matmul():
    ops = Operations()
    ops.input("A", shape=(32, 64))
    ops.input("B", shape=(64, 64))
    ops.input("bias", shape=(1, 64))
    ops.elementwise("exp", out="A_exp", operands=("A",))
    ops.matmul(a="A_exp", b="B", out="C")
    ops.elementwise("add", out="D", operands=("C", "bias"), y_broadcast="row")
    ops.elementwise("max", out="Y", operands=("D", 0.0))
    (v,) = fuse(ops.build())
    assert _types(v) == ["ElementwiseOp", "MatmulOp", "ElementwiseOp", "ElementwiseOp"]
    pre, post = _around_anchor(v)
    assert [op.op for op in pre] == ["exp"] and len(post) == 2
    assert assemble(v).strategy is FusionStrategy.MATMUL_EPILOGUE_TG


def test_multi_consumer_output_blocks_epilogue():
    ops = Operations()
    ops.input("A", shape=(64, 64))
    ops.input("B", shape=(64, 64))
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("exp", out="D", operands=("C",))
    ops.elementwise("log", out="E", operands=("C",))
    strategies = [assemble(v).strategy for v in fuse(ops.build())]
    assert FusionStrategy.STANDALONE_MATMUL in strategies
    elem = {FusionStrategy.STANDALONE_ELEMENTWISE, FusionStrategy.ELEMENTWISE_CHAIN}
    assert sum(s in elem for s in strategies) == 2


def test_shared_lane_agnostic_prologue_is_recomputed_and_elided():
    ops = Operations()
    ops.input("X", shape=(64, 64))
    ops.input("B1", shape=(64, 64))
    ops.input("B2", shape=(64, 64))
    ops.elementwise("max", out="Xr", operands=("X", 0.0))
    ops.matmul(a="Xr", b="B1", out="C1")
    ops.matmul(a="Xr", b="B2", out="C2")
    vs = fuse(ops.build())
    mm = [v for v in vs if any(isinstance(op, MatmulOp) for op in v.ops)]
    assert len(mm) == 2
    for v in mm:
        assert [op.op for op in _around_anchor(v)[0]] == ["max"]
    assert [v for v in vs if all(isinstance(op, ElementwiseOp) for op in v.ops)] == []


def test_shared_tensor_prologue_stays_materialised():
    ops = Operations()
    ops.input("X", shape=(64, 64))
    ops.input("bias", shape=(1, 64))
    ops.input("B1", shape=(64, 64))
    ops.input("B2", shape=(64, 64))
    ops.elementwise("add", out="Xb", operands=("X", "bias"), y_broadcast="row")
    ops.matmul(a="Xb", b="B1", out="C1")
    ops.matmul(a="Xb", b="B2", out="C2")
    vs = fuse(ops.build())
    mm = [v for v in vs if any(isinstance(op, MatmulOp) for op in v.ops)]
    assert len(mm) == 2
    for v in mm:
        assert _around_anchor(v)[0] == []
        assert assemble(v).strategy is FusionStrategy.STANDALONE_MATMUL
    assert len([v for v in vs if all(isinstance(op, ElementwiseOp) for op in v.ops)]) == 1


def _two_matmuls(shared: bool, n=32):
    ops = Operations()
    ops.input("A", shape=(n, n))
    if shared:
        ops.input("B1", shape=(n, n))
        ops.input("B2", shape=(n, n))
        ops.matmul(a="A", b="B1", out="c1")
        ops.matmul(a="A", b="B2", out="c2")
    else:
        for name in "BCD":
            ops.input(name, shape=(n, n))
        ops.matmul(a="A", b="B", out="c1")
        ops.matmul(a="C", b="D", out="c2")
    ops.elementwise("add", out="z", operands=("c1", "c2"))
    return ops


def test_multi_producer_and_diamond_labels():
    (v,) = fuse(_two_matmuls(False).build())
    assert _types(v) == ["MatmulOp", "MatmulOp", "ElementwiseOp"]
    assert assemble(v).strategy is FusionStrategy.MULTI_PRODUCER_CONVERGENT
    (v,) = fuse(_two_matmuls(True).build())
    assert assemble(v).strategy is FusionStrategy.DIAMOND_SHARED


def test_multi_producer_kernel_structure():
    """Reference: two suffixed accumulator sets, two C tiles, A0/A1 tiles.
    gfx950: two register accumulator sets ``acc_0``/``acc_1`` merged per
    register (no C tiles), A0/A1 and B0/B1 LDS tiles."""
    g = assemble(fuse(_two_matmuls(False).build())[0])
    src = g.kernel.source
    assert "acc_0" in src and "acc_1" in src
    assert "merge(acc_0[i][j][v], acc_1[i][j][v])" in src
    assert g.bindings == ("A", "B", "C", "D", "z")
    assert src.count("__shared__ alignas(16) float A0_tile") == 1
    assert src.count("__shared__ alignas(16) float A1_tile") == 1
    assert "C0_tile" not in src


def test_diamond_kernel_structure():
    g = assemble(fuse(_two_matmuls(True).build())[0])
    src = g.kernel.source
    assert "__shared__ alignas(16) float A_tile" in src
    assert "A0_tile" not in src and "A1_tile" not in src
    assert "B0_tile" in src and "B1_tile" in src
    assert "acc_0" in src and "acc_1" in src
    assert g.bindings == ("A", "B1", "B2", "z")
    assert g.dims == (32, 32, 32)


def test_reduction_output_never_feeds_matmul():
    ops = Operations()
    ops.input("X", shape=(8, 16))
    ops.input("A", shape=(8, 16))
    ops.input("B", shape=(16, 8))
    ops.reduction("sum", out="R", x="X")
    ops.matmul(a="A", b="B", out="C")
    strategies = {assemble(v).strategy for v in fuse(ops.build())}
    assert {FusionStrategy.STANDALONE_REDUCTION, FusionStrategy.STANDALONE_MATMUL} <= strategies


def test_bias_relu_kernel_text():
    """Reference: simdgroup MMA, bias staged in eY0_tile, fmax chain on
    C_tile, output at buffer(2), bias as extra device input.
    gfx950: MFMA tile call, bias read per register in the epilogue
    (``g_bias[col]``), fmaxf in the epilogue helper, output third param."""
    g = assemble(fuse(_bias_relu().build())[0])
    src = g.kernel.source
    assert "mt_mfma_tile<" in src
    assert "epilogue(acc[i][j][v], g_bias[(size_t)(col)])" in src
    assert "fmaxf" in src
    params = src.split("__launch_bounds__")[1].split("{")[0]
    assert params.index("float* __restrict__ g_Y") > params.index("g_B")
    assert "const float* __restrict__ g_bias" in src
    assert g.bindings == ("A", "B", "Y", "bias")


def test_register_epilogue_text():
    """Reference: thread_elements() per-lane writes.  gfx950: the epilogue
    helper applied to every accumulator register before the store."""
    ops = Operations()
    ops.input("A", shape=(128, 64))
    ops.input("B", shape=(64, 128))
    ops.matmul(a="A", b="B", out="C")
    ops.elementwise("max", out="Y", operands=("C", 0.0))
    g = assemble(fuse(ops.build())[0])
    assert g.strategy is FusionStrategy.MATMUL_EPILOGUE_REGISTER
    assert "epilogue(acc[i][j][v])" in g.kernel.source and "fmaxf" in g.kernel.source


def test_where_reads_cond_operand():
    ops = Operations()
    for name in ("X", "Y", "Cond"):
        ops.input(name, shape=(16, 16))
    ops.elementwise("where", out="Z", operands=("X", "Y", "Cond"))
    g = assemble(fuse(ops.build())[0])
    assert g.bindings == ("X", "Z", "Y", "Cond")
    src = g.kernel.source
    assert "const float* __restrict__ g_Cond" in src
    assert "(e1) != 0.0f ? (s0) : (e0)" in src


def test_1d_elementwise_is_m_by_1():
    ops = Operations()
    ops.input("X", shape=(128,))
    ops.elementwise("exp", out="Y", operands=("X",))
    g = assemble(fuse(ops.build())[0])
    assert g.dims == (128, 1)
    # gfx950 flat layout: 128 floats fit one workgroup
    assert g.grid == (1, 1, 1)


def test_same_input_twice_binds_once():
    ops = Operations()
    ops.input("X", shape=(16, 16))
    ops.elementwise("mul", out="Y", operands=("X", "X"))
    g = assemble(fuse(ops.build())[0])
    assert g.bindings == ("X", "Y")
    assert g.kernel.source.count("const float* __restrict__ g_X") == 1


def test_in_chain_secondary_reuses_register():
    ops = Operations()
    ops.input("X", shape=(16, 16))
    ops.elementwise("exp", out="E", operands=("X",))
    ops.elementwise("add", out="Y", operands=("E", "E"))
    (v,) = fuse(ops.build())
    assert _types(v) == ["ElementwiseOp", "ElementwiseOp"]
    g = assemble(v)
    src = g.kernel.source
    assert g.bindings == ("X", "Y") and "g_E" not in src
    assert "const float v0 = expf((s0));" in src
    assert "const float v1 = (v0) + (v0);" in src


def test_secondary_view_reads_through_strides():
    ops = Operations()
    ops.input("X", shape=(4, 8))
    ops.input("Ybase", shape=(8, 4))
    ops.transpose("Ybase", out="Y")
    ops.elementwise("add", out="Z", operands=("X", "Y"))
    g = assemble(fuse(ops.build())[0])
    assert g.bindings == ("X", "Z", "Ybase")
    # Y has strides (1, 4): column steps of 4 elements
    assert "g_Ybase[(size_t)(row) + (size_t)(col + 1u) * 4u]" in g.kernel.source
